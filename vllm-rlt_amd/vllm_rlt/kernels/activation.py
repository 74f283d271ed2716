"""SiLU-and-Mul on the gfx950 C ABI (``vrh_silu_and_mul``).

Operator contract of the reference's ``vllm_rlt/kernels/activation.py:9-33``
and its native entry ``csrc/activation/silu_and_mul.cu:221-245``:

* ``gate`` and ``up`` have the same shape (no broadcasting: ``ValueError``),
  device (``ValueError``) and dtype (``TypeError``); float32, float16 and
  bfloat16 only (``TypeError``);
* the native entry takes contiguous inputs only and copies nothing
  (``RuntimeError`` "contiguous inputs"); storage offsets may be misaligned;
* inference only: inputs that require grad with grad mode on raise
  ``RuntimeError`` ("inference-only");
* the result owns new storage with the inputs' shape, dtype and device; SiLU
  is rounded to the dtype before the multiply, as ``F.silu(gate) * up``.

There is no CPU path: this is the ``hip`` build, and non-ROCm tensors raise
``ValueError``.
"""

from __future__ import annotations

import torch

from vllm_rlt.kernels._hip import VRH_DTYPE_BF16, VRH_DTYPE_F16, VRH_DTYPE_F32, library

_CODES = {torch.float32: VRH_DTYPE_F32, torch.float16: VRH_DTYPE_F16,
          torch.bfloat16: VRH_DTYPE_BF16}


def _validate_inputs(gate: torch.Tensor, up: torch.Tensor) -> None:
    if gate.shape != up.shape:
        raise ValueError("silu_and_mul expects inputs with the same shape")
    if gate.device != up.device:
        raise ValueError("silu_and_mul expects inputs on the same device")
    if gate.dtype != up.dtype:
        raise TypeError("silu_and_mul expects inputs with the same dtype")
    if gate.dtype not in _CODES:
        raise TypeError("silu_and_mul supports float32, float16 and bfloat16")


def silu_and_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``F.silu(gate) * up`` with the SiLU rounded to the dtype, on the gfx950 kernel."""
    _validate_inputs(gate, up)
    if gate.device.type != "cuda":
        raise ValueError("silu_and_mul of the hip build needs ROCm device tensors")
    if not (gate.is_contiguous() and up.is_contiguous()):
        raise RuntimeError("silu_and_mul expects contiguous inputs")
    if torch.is_grad_enabled() and (gate.requires_grad or up.requires_grad):
        raise RuntimeError(
            "silu_and_mul is inference-only; use torch.no_grad() or silu_and_mul_reference")
    out = torch.empty(gate.shape, dtype=gate.dtype, device=gate.device)
    count = gate.numel()
    if count == 0:
        return out
    lib = library()
    lib.check(
        lib.vrh_silu_and_mul(_CODES[gate.dtype], out.data_ptr(), gate.data_ptr(), up.data_ptr(),
                             count, torch.cuda.current_stream(gate.device).cuda_stream),
        "vrh_silu_and_mul",
    )
    return out
