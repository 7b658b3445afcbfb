// Checks of the benchmark driver's building blocks that need no GPU (test infrastructure):
//  - SHA-256 known answers (FIPS 180-4 examples; the reference's tests/Native.cpp:18-22 pins
//    sha256("abc")), including inputs that cross the 64-byte block and padding boundaries;
//  - nearest-rank percentiles (the reference's tests/test_analysis.py:9-12);
//  - the Errors thresholds at their edges, FP32 and mixed (bench/Main.cpp:57-84);
//  - JSON round trips and equality as the driver uses them, and the parser's rejections:
//    numbers outside the JSON grammar, unpaired surrogates, nesting beyond its limit.
// With the argument "halves" it prints the FP32 bits of every FP16 bit pattern's decode, one
// hex word per line, for the Python test to compare with numpy; with "fuzz N" it feeds N
// mutated documents to the JSON parser (for the sanitizer builds).
#include "json.hpp"
#include "metrics.hpp"
#include "model.hpp"
#include "sha256.hpp"

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

using namespace stbench;

static int failures = 0;
static void expect(bool ok, const char* what) {
  if (!ok) {
    failures++;
    std::printf("FAIL %s\n", what);
  }
}

// Random mutations of valid documents (byte flips, truncations, insertions of structural
// characters) through the parser: each must parse or throw std::runtime_error; under the
// address and undefined-behaviour sanitizers any out-of-bounds read or overflow aborts.
static int fuzz(unsigned rounds) {
  const std::vector<std::string> seeds{
      R"({"version": 1, "config": {"layers": 2, "epsilon": 1e-05}, "tensors": [{"name": "x", "offset": 0}]})",
      R"([1, -2.5e+3, "a\u00e9\ud83d\ude00", true, false, null, {"k": [[], {}]}])",
      R"({"state_events": [0, 64, 128], "sha256": "00ff", "n": 18446744073709551615})"};
  uint64_t x = 0x9E3779B97F4A7C15ull;
  auto next = [&]() {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return x;
  };
  const char alphabet[] = "{}[],:\"\\0123456789.eE+-tfnu ";
  unsigned parsed = 0;
  for (unsigned r = 0; r < rounds; r++) {
    std::string doc = seeds[next() % seeds.size()];
    const unsigned edits = 1 + next() % 4;
    for (unsigned e = 0; e < edits && !doc.empty(); e++) {
      const size_t at = next() % doc.size();
      switch (next() % 4) {
        case 0: doc[at] = alphabet[next() % (sizeof alphabet - 1)]; break;
        case 1: doc.erase(at, 1 + next() % 3); break;
        case 2: doc.insert(at, 1, alphabet[next() % (sizeof alphabet - 1)]); break;
        default: doc.resize(at); break;
      }
    }
    try {
      const Json j = Json::parse(doc);
      (void)j.dump(2);
      parsed++;
    } catch (const std::runtime_error&) {
    }
  }
  std::printf("fuzz: %u rounds, %u parsed\n", rounds, parsed);
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 2 && std::string(argv[1]) == "fuzz") return fuzz((unsigned)std::stoul(argv[2]));
  if (argc > 1 && std::string(argv[1]) == "halves") {
    for (unsigned h = 0; h < 65536; h++) {
      const float f = half_to_float((uint16_t)h);
      uint32_t bits;
      std::memcpy(&bits, &f, 4);
      std::printf("%08x\n", bits);
    }
    return 0;
  }
  expect(sha256("abc", 3) == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad", "sha256(abc)");
  expect(sha256("", 0) == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855", "sha256(empty)");
  const char* two = "abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq";
  expect(sha256(two, std::strlen(two)) == "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1",
         "sha256(448-bit message)");
  std::vector<char> million(1000000, 'a');
  Sha256 incremental;
  for (size_t i = 0; i < million.size(); i += 997) incremental.update(million.data() + i, std::min<size_t>(997, million.size() - i));
  expect(incremental.hex() == "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0",
         "sha256(one million 'a', fed in 997-byte pieces)");

  std::vector<double> v;
  for (int i = 1; i <= 100; i++) v.push_back(i);
  Json d = distribution(v);
  expect(d.at("p50_us").number() == 50 && d.at("p95_us").number() == 95 && d.at("p99_us").number() == 99 &&
             d.at("p999_us_diagnostic").number() == 100 && d.at("worst_us").number() == 100,
         "nearest-rank percentiles of 1..100");
  expect(distribution({7.0}).at("p50_us").number() == 7 && distribution({}).size() == 0, "one sample / no samples");

  Errors e;
  e.check(1.0f, 1.0f, false);
  e.check(1.0f + 1.05e-4f, 1.0f, false);  // within 1e-5 + 1e-4
  e.check(1.0f + 1.2e-4f, 1.0f, false);   // beyond
  e.check(NAN, 1.0f, false);
  expect(e.count == 4 && e.failed == 2 && e.nonfinite == 1, "FP32 thresholds and non-finite values");
  Errors m;
  m.check(0.0f, 0.0f, true, 3);
  m.check(5.9e-3f, 0.0f, true, 3);   // within 2e-3 * 3
  m.check(6.1e-3f, 0.0f, true, 3);   // beyond
  m.check(10.2f, 10.0f, true, 1);    // within 2e-3 + 2e-2 * 10
  m.check(10.3f, 10.0f, true, 1);    // beyond
  expect(m.count == 5 && m.failed == 2, "mixed thresholds with the absolute scale");
  const float ref[4] = {3, 4, 0, 0}, act[4] = {3, 4, 0, 1};
  expect(std::fabs(relative_l2(act, ref, 4) - 0.2) < 1e-12 && residual_scale(ref, 4) == 2.5 &&
             mixed_state_scale(ref, 4, 2) == 7.5,
         "relative L2, residual scale and the mixed state scale");

  const Json j = Json::parse(R"({"b": [1, 2.5, -3, true, null, "x\"yé"], "a": {"n": 18446744073709551615}})");
  expect(j.at("a").at("n").uinteger() == 18446744073709551615ull, "64-bit unsigned integers");
  expect(Json::parse(j.dump(2)) == j && Json::parse(j.dump()) == j, "dump / parse round trip");
  expect(Json::parse(R"({"x": 1, "y": 1e-05})") == Json::parse(R"({"y": 0.00001, "x": 1})"), "object equality");
  expect(Json::parse("[1]") != Json::parse("[1.5]"), "number inequality");
  auto rejected = [](const std::string& text) {
    try {
      Json::parse(text);
    } catch (const std::runtime_error&) {
      return true;
    }
    return false;
  };
  expect(rejected("{\"a\": 1,}"), "malformed JSON rejected");
  // Numbers are checked against the JSON grammar as a whole token: no prefix parses.
  for (const char* bad : {"12-3", "1+", "01", "-", "1.", ".5", "1e", "1e+", "--1", "[1-2]", "0x10", "+1"})
    expect(rejected(bad), bad);
  expect(Json::parse("-0").integer() == 0 && Json::parse("1E+2").number() == 100 && Json::parse("-12").integer() == -12 &&
             Json::parse("2.5e-1").number() == 0.25,
         "numbers in the grammar");
  // Doubles beyond the range are errors; underflow rounds to a subnormal or zero; integers
  // beyond 64 bits keep their double value.
  expect(rejected("1e99999") && rejected("[-1.5e400]"), "overflowing numbers rejected");
  expect(Json::parse("1e-400").number() == 0.0 && Json::parse("4.9e-324").number() > 0.0, "underflow");
  expect(Json::parse("123456789012345678901234567890").number() == 123456789012345678901234567890.0, "wide integer");
  // Surrogate pairs: a high surrogate needs a following low one; a lone low one is an error.
  expect(Json::parse(R"("\ud83d\ude00")").str() == "\xF0\x9F\x98\x80", "surrogate pair decodes to U+1F600");
  for (const char* bad : {R"("\ud83d")", R"("\ud83dx")", R"("\ud83dA")", R"("\ud83d\ud83d")", R"("\ude00")"})
    expect(rejected(bad), bad);
  // Nesting depth is bounded.
  expect(!rejected(std::string(200, '[') + std::string(200, ']')), "200 levels of nesting");
  expect(rejected(std::string(100000, '[') + std::string(100000, ']')), "100000 levels of nesting rejected");

  std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "OK", failures);
  return failures ? 1 : 0;
}
