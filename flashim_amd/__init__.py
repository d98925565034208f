"""flashim_amd: an MI355X (gfx950) backend for FlashIM's quantized implicit-GEMM convolution path.

Hand-written HIP kernels (``flashim_amd/csrc``) behind a C ABI (``include/flashim_amd.h``), called through ctypes on
PyTorch's current stream, registered behind FlashIM's op plugin API (:mod:`flashim_amd.ops`, or into FlashIM itself
through :mod:`flashim_amd.plugin`).
"""

from flashim_amd import ops, quant  # noqa: F401

__version__ = "0.1.0"
