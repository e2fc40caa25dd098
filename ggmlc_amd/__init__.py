"""ggmlc_amd — MI355X (gfx950) implementation of ggmlc's quantized execution hot path.

The product is ``libgq.so`` (HIP kernels behind the C ABI of ``include/gq.h``);
``ggmlc_amd.ops`` calls it on torch device tensors. See ``ops`` for the
operator list and ``_lib`` for the binding.
"""

from ._lib import GQError, LIB_PATH  # noqa: F401

__version__ = "0.1.0"


def get_available_devices() -> list[str]:
    """Devices this runtime can execute on (mirrors ggmlc runtime/runner.py:34-38).

    Only GPUs are listed: the quantized path here has no CPU implementation."""
    try:
        import torch

        if torch.cuda.is_available():
            return [f"gpu:{i}" for i in range(torch.cuda.device_count())]
    except Exception:  # pragma: no cover - torch import failure
        pass
    return []
