"""Host side of the MI355X streaming-step backend (libstamd.so).

streamtx.model    checkpoint format, config validation, synthetic checkpoints
streamtx.runtime  ctypes binding of the C ABI (include/st_runtime.h), mirroring Stream::Runtime
streamtx.numerical acceptance metrics of the reference (include/Numerical.hpp, reference/numerical.py)
streamtx.build    hipcc build of libstamd.so for gfx950
"""
from .model import (Checkpoint, ModelConfig, load_checkpoint, round_bf16, round_half, synthetic_checkpoint,
                    tensor_names, write_checkpoint)
from .runtime import Backend, BatchRuntime, Runtime, RuntimeOptions, WeightStorage, library, probe, transport_bench

__all__ = ['Backend', 'BatchRuntime', 'Checkpoint', 'ModelConfig', 'Runtime', 'RuntimeOptions', 'WeightStorage', 'library',
           'load_checkpoint', 'probe', 'transport_bench', 'round_bf16', 'round_half', 'synthetic_checkpoint', 'tensor_names',
           'write_checkpoint']
