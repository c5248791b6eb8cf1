"""fellm_amd — MI355X (gfx950) kernels for FeLLM's per-layer memory-bound ops.

Layers:
  * ``libfellm_rocm_kernels.so`` (csrc/): hand-written HIP kernels plus the
    FeLLM plugin C ABI (include/fellm_abi.h) and a device-pointer API
    (include/fellm_rocm.h).
  * ``fellm_amd.plugin_host``: a Python restatement of fellm-plugin-host
    (dlopen, ABI check, registry keyed by (op, dtypes), launch).
  * ``fellm_amd.ops``: torch-tensor wrappers over the device-pointer API.
"""
from . import abi  # noqa: F401
from ._lib import EXPORTED, LIB_PATH, FellmRocmError, lib  # noqa: F401

__version__ = "0.1.0"
