"""Load the torch operator library ``vllm_rlt._C`` once.

Same contract as the reference's ``vllm_rlt/kernels/_extension.py:7-23``:
``try_load_extension()`` imports the module once and caches whether it was
found; ``load_extension()`` raises when it is missing. Importing the module
registers ``torch.ops.vllm_rlt.silu_and_mul`` (the reference's op) and the
paged-KV ops under ``torch.ops.vllm_rlt_hip`` (CUDA dispatch key only: ROCm
tensors). The module is built with the gfx950 library (``make`` in
``vllm-rlt_amd``) and forwards to it.
"""

from functools import cache
from importlib import import_module


@cache
def try_load_extension() -> bool:
    """Import once; a missing module is cached as unavailable."""
    try:
        import_module("vllm_rlt._C")
    except ModuleNotFoundError as exc:
        if exc.name != "vllm_rlt._C":
            raise
        return False
    return True


def load_extension() -> None:
    if not try_load_extension():
        raise RuntimeError(
            "The torch operator library vllm_rlt._C is not built: run make in vllm-rlt_amd.")
