// Host-side checks of the batched projections' operand layouts (test infrastructure), compiled
// with hipcc from the library's own header: act_index (FP32 buffers, for the FP32 MFMA and for
// the bfloat16 MFMA) and half_index (FP16 buffers). What the kernels rely on:
//  - each layout is a bijection from [0, rows) x [0, cols) onto [0, rows * cols);
//  - a 16-row x KB-column block of the operand is one contiguous run, its 64 lanes in order,
//    lane l holding row (b mod 16) = l mod 16 and consecutive columns of column group l / 16
//    (4 per lane for KB = 16; 8 per lane for KB = 32, as two planes of 4 for FP32 and 8
//    consecutive halves for FP16);
//  - four consecutive columns from a multiple of 4 are consecutive in memory.
#include "../streaming-transformer_amd/csrc/step_device.hpp"
#include "../streaming-transformer_amd/csrc/batch_kernels.hpp"

#include <cstdio>
#include <functional>
#include <vector>

using namespace stamd;

static int failures = 0;
static void expect(bool ok, const char* what, int rows, int cols) {
  if (!ok) {
    failures++;
    std::printf("FAIL %s (rows %d, cols %d)\n", what, rows, cols);
  }
}

// kb: columns per block; per_lane: values per lane; planes: how a lane's values are split.
static void check(const char* name, const std::function<size_t(int, int, int)>& index, int kb, int per_lane,
                  int planes) {
  for (int rows : {16, 32, 64, 256})
    for (int cols : {32, 64, 256, 512, 1024, 4096}) {
      std::vector<int> seen((size_t)rows * cols, 0);
      bool in_range = true, blocks = true, lanes = true, runs = true;
      for (int b = 0; b < rows; b++)
        for (int n = 0; n < cols; n++) {
          const size_t i = index(b, n, cols);
          if (i >= seen.size()) {
            in_range = false;
            continue;
          }
          seen[i]++;
          // The block (b / 16, n / kb) is the run [block * 16 kb, (block + 1) * 16 kb).
          const size_t block = (size_t)(b / 16) * (cols / kb) + n / kb;
          if (i / (16 * kb) != block) blocks = false;
          // Within it: plane, then lane, then the lane's values.
          const size_t at = i % (16 * kb), per_plane = per_lane / planes;
          const int plane = (int)(at / (64 * per_plane)), lane = (int)(at % (64 * per_plane) / per_plane);
          const int value = (int)(at % per_plane) + plane * (int)per_plane;
          const int group = (n % kb) / per_lane;
          if (lane != b % 16 + 16 * group || value != (n % kb) % per_lane) lanes = false;
          if (n % 4 == 0)
            for (int j = 1; j < 4; j++)
              if (index(b, n + j, cols) != i + j) runs = false;
        }
      bool bijective = in_range;
      for (int v : seen) bijective = bijective && v == 1;
      std::printf("%s rows %d cols %d: bijective %d blocks %d lanes %d runs %d\n", name, rows, cols, bijective, blocks,
                  lanes, runs);
      expect(bijective, "bijection", rows, cols);
      expect(blocks, "16 x KB blocks are contiguous runs", rows, cols);
      expect(lanes, "lane l holds row l mod 16 and its column group's consecutive values", rows, cols);
      expect(runs, "four consecutive columns are consecutive", rows, cols);
    }
}

int main() {
  check("fp32 (FP32 MFMA)", [](int b, int n, int c) { return act_index<kFp32>(b, n, c); }, 16, 4, 1);
  check("fp32 (bfloat16 MFMA)", [](int b, int n, int c) { return act_index<kBf16w>(b, n, c); }, 32, 8, 2);
  check("fp32 x (mixed mode)", [](int b, int n, int c) { return act_index<kMixed>(b, n, c); }, 16, 4, 1);
  check("fp16", [](int b, int n, int c) { return half_index(b, n, c); }, 32, 8, 1);
  std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "OK", failures);
  return failures ? 1 : 0;
}
