"""tbf16 for MI355X: bf16 matmuls and attention on fp16 MFMA with exact power-of-two scaling.

Drop-in for tech-cosmos/turing-bf16's public API (tbf16/__init__.py:3-11 there):
same names, signatures and results, with hand-written gfx950 HIP kernels behind a
C ABI (include/tbf16_hip.h) instead of CUDA/Triton.
"""
__version__ = "0.1.0"

from .attention import sdpa
from . import autograd
from .convert import Linear, TrainLinear, convert, install_sdpa, is_supported_gpu, uninstall_sdpa
from .ops import prepare_weight, quantize_rows, scaled_linear
from .patch import TuringBF16Mode, patch

__all__ = ["quantize_rows", "scaled_linear", "prepare_weight", "sdpa", "patch", "TuringBF16Mode", "convert",
           "Linear", "TrainLinear", "autograd", "install_sdpa", "uninstall_sdpa",
           "is_supported_gpu"]
