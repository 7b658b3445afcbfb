"""Model contract: configuration, checkpoint format and synthetic checkpoints.

Host-side counterpart of Stream::ModelConfig / Stream::Model (include/Model.hpp:12-35,
src/runtime/Model.cpp:15-139). The on-disk format is the reference's unchanged:
``manifest.json`` (version 1, little endian, ``out_in`` orientation, per-tensor and
archive SHA256) plus ``tensors.bin`` (reference/export.py:31-43), so checkpoints written
by the reference and by :func:`write_checkpoint` load the same way.
"""
from __future__ import annotations

import hashlib
import json
from dataclasses import asdict, dataclass
from pathlib import Path

import numpy as np

__all__ = ['ModelConfig', 'Checkpoint', 'load_checkpoint', 'write_checkpoint', 'synthetic_checkpoint',
           'tensor_names', 'round_half', 'round_bf16']


@dataclass(frozen=True)
class ModelConfig:
    """The seven model fields (include/Model.hpp:12-18)."""
    layers: int
    width: int
    heads: int
    ffn: int
    window: int
    features: int
    epsilon: float = 1e-5

    def validate(self) -> 'ModelConfig':
        """ModelConfig::validate (src/runtime/Model.cpp:22-29); raises ValueError."""
        c = self
        bad = (c.layers < 1 or c.layers > 16 or c.width < 1 or c.width > 1024 or c.heads < 1
               or c.width % c.heads or (c.width // c.heads) % 2 or c.ffn < 1 or c.ffn > 4096
               or c.window < 1 or c.window > 4096 or c.features < 1 or c.features > 1024
               or not np.isfinite(c.epsilon) or c.epsilon <= 0)
        if bad:
            raise ValueError('Invalid or unsupported model dimensions')
        return self

    @property
    def dim(self) -> int:
        return self.width // self.heads

    def cache_elements(self) -> int:
        """ModelConfig::cacheElements (src/runtime/Model.cpp:31-33)."""
        return self.layers * self.width * self.window

    @classmethod
    def from_json(cls, obj: dict) -> 'ModelConfig':
        return cls(int(obj['layers']), int(obj['width']), int(obj['heads']), int(obj['ffn']),
                   int(obj['window']), int(obj['features']), float(obj['epsilon'])).validate()

    def to_json(self) -> dict:
        return asdict(self)


def tensor_names(config: ModelConfig) -> list[tuple[str, tuple[int, ...]]]:
    """Tensor names and shapes in checkpoint order (reference/model.py:27-47)."""
    c = config
    out = [('input', (c.width, c.features))]
    for layer in range(c.layers):
        p = f'layers.{layer}.'
        out += [(p + 'norm1', (c.width,)), (p + 'norm2', (c.width,))]
        out += [(p + n, (c.width, c.width)) for n in ('q', 'k', 'v', 'out')]
        out += [(p + 'gate', (c.ffn, c.width)), (p + 'up', (c.ffn, c.width)), (p + 'down', (c.width, c.ffn))]
    out += [('final_norm', (c.width,)), ('score', (1, c.width))]
    return out


@dataclass
class Checkpoint:
    config: ModelConfig
    mixed: bool
    tensors: dict  # name -> float32 ndarray (FP16 files decoded)
    manifest: dict


def _sha256(raw: bytes) -> str:
    return hashlib.sha256(raw).hexdigest()


def load_checkpoint(path) -> Checkpoint:
    """Stream::Model::Model (src/runtime/Model.cpp:63-140): format, hashes, bounds, shapes."""
    path = Path(path)
    manifest = json.loads((path / 'manifest.json').read_text())
    if (manifest.get('version') != 1 or manifest.get('byte_order') != 'little'
            or manifest.get('orientation') != 'out_in'):
        raise ValueError('Unsupported tensor format')
    config = ModelConfig.from_json(manifest['config'])
    mode = manifest['mode']
    if mode not in ('fp32', 'mixed'):
        raise ValueError('Unknown numerical mode')
    raw = (path / 'tensors.bin').read_bytes()
    if _sha256(raw) != manifest['sha256']:
        raise ValueError('Checkpoint hash mismatch')
    tensors, end = {}, 0
    for item in manifest['tensors']:
        shape = tuple(int(d) for d in item['shape'])
        if any(d <= 0 for d in shape):
            raise ValueError('Invalid tensor dimensions')
        count = int(np.prod(shape))
        size = {'float32': 4, 'float16': 2}.get(item['dtype'], 0)
        offset, nbytes = int(item['offset']), int(item['nbytes'])
        if not size or offset != end or nbytes != count * size or offset + nbytes > len(raw):
            raise ValueError('Invalid tensor bounds')
        part = raw[offset:offset + nbytes]
        if _sha256(part) != item['sha256']:
            raise ValueError('Tensor hash mismatch')
        dtype = '<f4' if size == 4 else '<f2'
        if item['name'] in tensors:
            raise ValueError('Duplicate tensor')
        tensors[item['name']] = np.frombuffer(part, dtype=dtype).astype(np.float32).reshape(shape)
        end += nbytes
    if end != len(raw):
        raise ValueError('Trailing tensor bytes')
    for name, shape in tensor_names(config):
        if name not in tensors or tensors[name].shape != shape:
            raise ValueError(f'Shape mismatch: {name}')
    return Checkpoint(config, mode == 'mixed', tensors, manifest)


def write_checkpoint(path, config: ModelConfig, tensors: dict, mixed: bool = False, **extra) -> Path:
    """Write the reference manifest format (reference/export.py:31-43)."""
    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    data = bytearray()
    manifest = dict(version=1, byte_order='little', orientation='out_in', config=config.to_json(),
                    mode='mixed' if mixed else 'fp32', **extra, tensors=[])
    for name, _shape in tensor_names(config):
        a = np.ascontiguousarray(tensors[name], dtype='<f2' if mixed else '<f4')
        raw = a.tobytes()
        manifest['tensors'].append(dict(name=name, shape=list(a.shape), dtype=str(a.dtype.name),
                                        offset=len(data), nbytes=len(raw), sha256=_sha256(raw)))
        data.extend(raw)
    manifest['sha256'] = _sha256(bytes(data))
    (path / 'tensors.bin').write_bytes(bytes(data))
    (path / 'manifest.json').write_text(json.dumps(manifest, indent=2) + '\n')
    return path


def round_half(x) -> np.ndarray:
    """Round to the nearest FP16 value (round to nearest even) and back to FP32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_bf16(x) -> np.ndarray:
    """Round to the nearest bfloat16 value (round to nearest even) and back to FP32."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7f800000) == 0x7f800000
    nan &= (u & 0x7fffff) != 0
    r = ((u + 0x7fff + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, (u | 0x400000) & 0xffff0000, r)
    return r.astype(np.uint32).view(np.float32)


def synthetic_checkpoint(config: ModelConfig, seed: int, std: float = 0.02, mixed: bool = False) -> dict:
    """Random-init weights of the reference architecture: matrices ~ N(0, std^2), norm
    weights 1 (reference/model.py:27-47 uses 1/sqrt(in) and seed 42; the benchmark
    configurations specify N(0, 0.02^2)). Deterministic in `seed` (numpy PCG64)."""
    config.validate()
    rng = np.random.default_rng(seed)
    tensors = {}
    for name, shape in tensor_names(config):
        if len(shape) == 1:
            t = np.ones(shape, dtype=np.float32)
        else:
            t = (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)
        tensors[name] = round_half(t) if mixed else t
    return tensors
