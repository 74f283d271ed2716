"""Select the paged attention implementation and declare its capabilities.

Same API as the reference's vllm_rlt/attention/backend.py:14-168
(``BackendCapabilities``, ``AttentionBackend``, ``create_backend``,
``validate_backend_name``, ``backend_capabilities``) with one GPU backend,
``hip`` (gfx950). The reference's own torch/triton/flash backends stay in the
reference; this build only adds ``hip``, and ``auto`` resolves to it.

Error contract (reference :148-152): construction failures are ``ValueError``
(unsupported device/dtype/head_dim/arch or missing capabilities) or
``ImportError``/``OSError`` (library missing or unloadable). Kernel-time errors
propagate; there is never a runtime fallback.
"""

from __future__ import annotations

import logging
from collections.abc import Callable
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class BackendCapabilities:
    """Features relevant to execution routing, independent of kernel class."""

    packed_prefill: bool = False
    cuda_graphs: bool = False
    async_scheduling: bool = False
    # Packed rows reproduce single-query decode bit for bit.
    packed_matches_decode: bool = False
    # Consume GPU-owned context lengths without a host read between submissions.
    device_context_lengths: bool = False
    # Mask keys outside a per-layer sliding window (not storage reclamation).
    sliding_window: bool = False


@dataclass
class AttentionBackend:
    """Thin kernel adapter with declared features and selection diagnostics."""

    kernel: Callable
    capabilities: BackendCapabilities
    info: dict

    def __call__(self, *args, **kwargs):
        return self.kernel(*args, **kwargs)

    def prefill(self, *args, **kwargs):
        return self.kernel.prefill(*args, **kwargs)

    def windowed(self, *args, **kwargs):
        method = getattr(self.kernel, "windowed", None)
        if method is None:
            selected = self.info.get("selected_backend", "this attention backend")
            raise NotImplementedError(f"{selected} does not implement sliding-window masking")
        return method(*args, **kwargs)

    @property
    def generation(self):
        return getattr(self.kernel, "generation", None)


HIP_CAPABILITIES = BackendCapabilities(
    packed_prefill=True,
    cuda_graphs=True,
    async_scheduling=True,
    # A packed call with max_seqlen_q <= PACKED_DECODE_EXACT_Q runs every query
    # as a split-KV decode row (the partition depends only on the row's own
    # length), so it reproduces single-query decode bit for bit; longer packed
    # sequences use MFMA tiles.
    packed_matches_decode=True,
    device_context_lengths=True,
    sliding_window=True,
)

# Largest max_seqlen_q for which packed rows equal single-query decode exactly
# (speculative verification packs draft + 1 tokens per request,
# worker/speculative.py:176-178).
PACKED_DECODE_EXACT_Q = 8

# Names the reference accepts; all but ``hip``/``auto`` belong to the reference.
_REFERENCE_ONLY = ("torch", "triton", "flash_attn", "flash_attn_2", "flash_attn_3",
                   "flash_attn_4")
_SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_SUPPORTED_ARCH = "gfx950"
_CAPABILITY_NAMES = ("packed_prefill", "cuda_graphs", "async_scheduling",
                     "device_context_lengths", "sliding_window")


def backend_capabilities(implementation) -> BackendCapabilities:
    return implementation.capabilities


def validate_backend_name(backend: str) -> None:
    if backend not in {"auto", "hip", *_REFERENCE_ONLY}:
        raise ValueError("unknown attention backend")


def _device_arch(device: torch.device) -> str:
    return torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]


def _create_explicit(backend, device, dtype, head_dim, block_size) -> AttentionBackend:
    if backend != "hip":
        raise ValueError(
            f"the {backend} attention backend belongs to vllm-rlt itself; this build provides hip"
        )
    if device.type != "cuda" or not torch.version.hip:
        raise ValueError("the hip attention backend requires a ROCm device")
    if dtype not in _SUPPORTED_DTYPES:
        raise ValueError("the hip attention backend supports float32, float16 and bfloat16")
    if not isinstance(head_dim, int) or not 0 < head_dim <= 256:
        raise ValueError("the hip attention backend supports head_dim <= 256")
    if not isinstance(block_size, int) or block_size <= 0:
        raise ValueError("block_size must be a positive integer")
    arch = _device_arch(device)
    if arch != _SUPPORTED_ARCH:
        raise ValueError(f"the hip attention backend is built for {_SUPPORTED_ARCH}, not {arch}")
    # Load (and ABI-check) the library now: ImportError/OSError if absent.
    from vllm_rlt.kernels._hip import library
    from vllm_rlt.kernels.hip_attention import HipPagedAttention

    library()
    return AttentionBackend(HipPagedAttention(), HIP_CAPABILITIES,
                            {"backend": "hip", "arch": arch,
                             "packed_matches_decode_max_seqlen_q": PACKED_DECODE_EXACT_Q})


def create_backend(
    backend: str,
    device: torch.device,
    dtype: torch.dtype,
    head_dim: int,
    block_size: int,
    *,
    required_capabilities: BackendCapabilities = BackendCapabilities(),
) -> AttentionBackend:
    """Explicit ``hip`` fails without fallback; ``auto`` selects ``hip`` when usable."""
    validate_backend_name(backend)
    device = torch.device(device)
    candidates = ("hip",) if backend == "auto" else (backend,)
    skipped = []
    for candidate in candidates:
        try:
            implementation = _create_explicit(candidate, device, dtype, head_dim, block_size)
            missing = [
                name
                for name in _CAPABILITY_NAMES
                if getattr(required_capabilities, name)
                and not getattr(implementation.capabilities, name)
            ]
            if missing:
                raise ValueError(f"{candidate} lacks required capabilities: {', '.join(missing)}")
        except (ValueError, ImportError, OSError) as error:
            if backend != "auto":
                raise
            skipped.append(f"{candidate}: {error}")
            continue
        reason = "auto selects the gfx950 hip backend" if backend == "auto" else (
            f"explicitly requested {backend}")
        implementation.info.update(
            requested_backend=backend, selected_backend=candidate, selection_reason=reason
        )
        logging.getLogger(__name__).info("Attention selection: %s", implementation.info)
        return implementation
    raise ValueError("no compatible attention backend; " + "; ".join(skipped))
