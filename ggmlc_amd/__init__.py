"""ggmlc_amd — MI355X (gfx950) implementation of ggmlc's quantized execution hot path.

The product is ``libgq.so`` (HIP kernels behind the C ABI of ``include/gq.h``);
``ggmlc_amd.ops`` calls it on torch device tensors. See ``ops`` for the
operator list and ``_lib`` for the binding.
"""

from ._lib import GQError, LIB_PATH  # noqa: F401

__version__ = "0.1.0"


def get_available_devices() -> list[str]:
    """Devices this runtime can execute on (mirrors ggmlc runtime/runner.py:34-38 and
    executor.cpp:184): the visible GPUs named as the reference names them, "cuda:N".

    Only GPUs are listed: the quantized path here has no CPU implementation."""
    from .runner import get_available_devices as _devs

    return _devs()
