"""Hidden-state row movement on the gfx950 C ABI (dtype-agnostic byte copies).

Mirrors the Triton kernels of the reference's ``kernels/routing.py``:
  gather_rows       gather_kernel (routing.py:51-66), called by
                    worker/async_state.py:104-113 and worker/async_speculative.py:371-380
  scatter_rows      scatter_kernel (routing.py:69-83), worker/async_state.py:115-123
  gather_segments   gather_segments_kernel (routing.py:86-113), worker/model_runner.py:515-552
  scatter_segments  scatter_segments_kernel (routing.py:116-144), worker/model_runner.py:554-597

Rows are the last dimension of 2-D tensors (contiguous rows, any row stride);
pool and batch tensors must share a dtype. Index tensors are int64 device
tensors. Launches go on the current stream; nothing synchronises.
"""

from __future__ import annotations

import torch

from vllm_rlt.kernels._hip import library


def _stream(tensor: torch.Tensor) -> int:
    return torch.cuda.current_stream(tensor.device).cuda_stream


def _rows(name: str, tensor: torch.Tensor, device: torch.device) -> None:
    if tensor.device.type != "cuda" or tensor.device != device:
        raise ValueError(f"{name} must be a ROCm device tensor on {device}")
    if tensor.ndim != 2 or tensor.stride(1) != 1:
        raise ValueError(f"{name} must be 2-D with contiguous rows")


def _index(name: str, tensor: torch.Tensor, device: torch.device, ndim: int) -> None:
    if tensor.device != device or tensor.dtype != torch.int64 or tensor.ndim != ndim:
        raise ValueError(f"{name} must be a {ndim}-D int64 tensor on {device}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _pair(a_name, a, b_name, b):
    device = a.device
    _rows(a_name, a, device)
    _rows(b_name, b, device)
    if a.dtype != b.dtype or a.shape[1] != b.shape[1]:
        raise ValueError(f"{a_name} and {b_name} must share dtype and row width")
    return device, a.shape[1] * a.element_size()


def gather_rows(pool: torch.Tensor, slots: torch.Tensor, out: torch.Tensor, n: int) -> torch.Tensor:
    """``out[r] = pool[slots[r]]`` for ``r < n`` and zeros for ``n <= r < len(out)``."""
    device, width = _pair("pool", pool, "out", out)
    _index("slots", slots, device, 1)
    size = out.shape[0]
    if not 0 <= n <= min(size, slots.shape[0]):
        raise ValueError("n must lie in [0, min(len(out), len(slots))]")
    lib = library()
    lib.check(
        lib.vrh_gather_rows(pool.data_ptr(), slots.data_ptr(), out.data_ptr(), n, size, width,
                            pool.stride(0) * pool.element_size(),
                            out.stride(0) * out.element_size(), _stream(out)),
        "vrh_gather_rows",
    )
    return out


def scatter_rows(values: torch.Tensor, slots: torch.Tensor, pool: torch.Tensor,
                 count: int | None = None) -> None:
    """``pool[slots[r]] = values[r]`` for ``r < count`` (default: every row of values)."""
    device, width = _pair("values", values, "pool", pool)
    _index("slots", slots, device, 1)
    count = values.shape[0] if count is None else count
    if not 0 <= count <= min(values.shape[0], slots.shape[0]):
        raise ValueError("count must lie in [0, min(len(values), len(slots))]")
    lib = library()
    lib.check(
        lib.vrh_scatter_rows(values.data_ptr(), slots.data_ptr(), pool.data_ptr(), count, width,
                             values.stride(0) * values.element_size(),
                             pool.stride(0) * pool.element_size(), _stream(pool)),
        "vrh_scatter_rows",
    )


def _segments(pool, segments, batch, pool_rows, max_rows):
    device, width = _pair("pool", pool, "batch", batch)
    _index("segments", segments, device, 2)
    if segments.shape[1] != 5:
        raise ValueError("segments must be [n, 5]: slot, row offset, count, batch start, keep")
    if pool_rows < 0 or max_rows < 0:
        raise ValueError("pool_rows and max_rows must be non-negative")
    return width


def gather_segments(pool: torch.Tensor, segments: torch.Tensor, out: torch.Tensor,
                    pool_rows: int, max_rows: int) -> torch.Tensor:
    """For each segment (slot, offset, count, start, keep): ``out[start + i] =
    pool[slot * pool_rows + offset + i]`` for ``i < count <= max_rows``."""
    width = _segments(pool, segments, out, pool_rows, max_rows)
    lib = library()
    lib.check(
        lib.vrh_gather_segments(pool.data_ptr(), segments.data_ptr(), out.data_ptr(),
                                segments.shape[0], max_rows, pool_rows, width,
                                pool.stride(0) * pool.element_size(),
                                out.stride(0) * out.element_size(), _stream(out)),
        "vrh_gather_segments",
    )
    return out


def scatter_segments(values: torch.Tensor, segments: torch.Tensor, pool: torch.Tensor,
                     pool_rows: int, max_rows: int) -> None:
    """The reverse of :func:`gather_segments` for segments whose ``keep`` is non-zero."""
    width = _segments(pool, segments, values, pool_rows, max_rows)
    lib = library()
    lib.check(
        lib.vrh_scatter_segments(values.data_ptr(), segments.data_ptr(), pool.data_ptr(),
                                 segments.shape[0], max_rows, pool_rows, width,
                                 values.stride(0) * values.element_size(),
                                 pool.stride(0) * pool.element_size(), _stream(pool)),
        "vrh_scatter_segments",
    )
