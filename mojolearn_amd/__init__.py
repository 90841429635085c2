"""mojolearn_amd: MI355X-native implementation of mojolearn's identical-mode FP32 GEMM/GEMV
(profile mojolearn.identical.gemm.fp32.v1, plus bf16- and int8-stored weights).

`mojolearn_amd.linalg` is the host-buffer surface of `mojolearn.linalg`; `mojolearn_amd.device`
takes PyTorch-ROCm device tensors.  Both call hand-written gfx950 kernels in libmlgemm.so
(C ABI: include/mlgemm.h).
"""
from . import linalg  # noqa: F401

__all__ = ["linalg", "device"]


def __getattr__(name):
    # `device` needs torch; import it on first use only
    if name == "device":
        import importlib
        return importlib.import_module(".device", __name__)
    raise AttributeError(name)
