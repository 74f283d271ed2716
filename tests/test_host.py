"""CPU tests of the host side: metadata planning (literal vectors from the
reference's tests/test_attention_module.py:45-131), backend selection errors
(attention/backend.py:102-168), host bookkeeping of the KV manager, and the
C-ABI library: it loads and exports every symbol include/vllm_rlt_hip.h
declares (no compute calls without a GPU)."""

import ctypes
import os
import re
from types import SimpleNamespace

import pytest
import torch

from vllm_rlt.attention import (
    AttentionRows,
    BackendCapabilities,
    backend_capabilities,
    build_attention_metadata,
    create_backend,
    plan_attention_metadata,
)
from vllm_rlt.kernels import _hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vllm_rlt_hip.h")


def test_metadata_is_depth_selected_padded():
    rows = AttentionRows(block_tables=[(4, 7, 8), (2, 3)], positions=[4, 1])
    metadata = build_attention_metadata(rows, block_size=2, device=torch.device("cpu"))
    assert metadata.block_tables.tolist() == [[4, 7, 8], [2, 3, -1]]
    assert metadata.context_lengths.tolist() == [5, 2]
    assert metadata.block_tables.dtype == metadata.context_lengths.dtype == torch.int32
    assert metadata.cu_seqlens_q is None
    assert metadata.max_seqlen_q == 1


def test_packed_metadata_groups_contiguous_query_chunks():
    rows = AttentionRows(
        block_tables=[(4, 7, 8), (4, 7, 8), (2, 3)],
        positions=[2, 3, 1],
        sequence_keys=[("a", 0), ("a", 0), ("b", 1)],
    )
    plan = plan_attention_metadata(rows, block_size=2, packed_prefill=True)
    assert plan.num_rows == 2
    assert plan.table_width == 2
    assert plan.block_tables == [4, 7, 2, 3]
    assert plan.context_lengths == [4, 2]
    assert plan.cu_seqlens_q == [0, 2, 3]
    assert plan.max_seqlen_q == 2


def test_packed_metadata_rejects_gaps_and_split_sequences():
    gap = AttentionRows(block_tables=[(1,), (1,)], positions=[0, 2],
                        sequence_keys=[("a", 0), ("a", 0)])
    with pytest.raises(ValueError, match="contiguous"):
        plan_attention_metadata(gap, block_size=4, packed_prefill=True)
    split = AttentionRows(block_tables=[(1,), (2,), (1,)], positions=[0, 0, 1],
                          sequence_keys=[("a", 0), ("b", 0), ("a", 0)])
    with pytest.raises(ValueError, match="one sequence"):
        plan_attention_metadata(split, block_size=4, packed_prefill=True)
    with pytest.raises(ValueError, match="sequence keys"):
        plan_attention_metadata(AttentionRows([(1,)], [0]), block_size=4, packed_prefill=True)
    with pytest.raises(ValueError, match="equal lengths"):
        plan_attention_metadata(AttentionRows([(1,)], [0, 1]), block_size=4)


def test_empty_plan():
    plan = plan_attention_metadata(AttentionRows([], []), block_size=16)
    assert plan.num_rows == 0 and plan.table_width == 0 and plan.block_tables == []


def test_backend_selection_errors_on_cpu():
    with pytest.raises(ValueError, match="unknown attention backend"):
        create_backend("unknown", torch.device("cpu"), torch.float32, 8, 2)
    with pytest.raises(ValueError, match="requires a ROCm device"):
        create_backend("hip", torch.device("cpu"), torch.float32, 8, 2)
    with pytest.raises(ValueError, match="no compatible attention backend"):
        create_backend("auto", torch.device("cpu"), torch.float32, 8, 2)
    with pytest.raises(ValueError, match="belongs to vllm-rlt"):
        create_backend("triton", torch.device("cpu"), torch.float32, 8, 2)


def test_backend_rejects_unsupported_configs_before_loading(monkeypatch):
    monkeypatch.setattr(torch.version, "hip", "7.0", raising=False)
    device = torch.device("cuda", 0)
    with pytest.raises(ValueError, match="float32, float16 and bfloat16"):
        create_backend("hip", device, torch.int8, 128, 16)
    with pytest.raises(ValueError, match="head_dim <= 256"):
        create_backend("hip", device, torch.bfloat16, 257, 16)
    monkeypatch.setattr(
        torch.cuda, "get_device_properties", lambda d: SimpleNamespace(gcnArchName="gfx942:sramecc+")
    )
    with pytest.raises(ValueError, match="built for gfx950"):
        create_backend("hip", device, torch.bfloat16, 128, 16)


def test_backend_reports_selection_and_capabilities(monkeypatch):
    monkeypatch.setattr(torch.version, "hip", "7.0", raising=False)
    monkeypatch.setattr(
        torch.cuda, "get_device_properties", lambda d: SimpleNamespace(gcnArchName="gfx950:sramecc+")
    )
    backend = create_backend("auto", torch.device("cuda", 0), torch.bfloat16, 128, 16,
                             required_capabilities=BackendCapabilities(packed_prefill=True,
                                                                       cuda_graphs=True))
    assert backend.info["selected_backend"] == "hip"
    assert backend.info["requested_backend"] == "auto"
    caps = backend_capabilities(backend)
    assert caps.packed_prefill and caps.cuda_graphs and caps.device_context_lengths
    assert caps.sliding_window and caps.packed_matches_decode
    assert backend.info["packed_matches_decode_max_seqlen_q"] == 8


def test_missing_library_is_an_import_error(monkeypatch, tmp_path):
    monkeypatch.setattr(_hip, "LIBRARY_PATH", str(tmp_path / "absent.so"))
    _hip.library.cache_clear()
    try:
        with pytest.raises(ImportError, match="not built"):
            _hip.library()
    finally:
        _hip.library.cache_clear()


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:[a-z_0-9]+\s*\*?\s+)+\**(vrh_[a-z_0-9]+)\s*\(", text,
                                 flags=re.M)))


def test_library_exports_every_declared_symbol():
    symbols = declared_symbols()
    assert "vrh_paged_decode" in symbols and "vrh_kv_append" in symbols and len(symbols) >= 12
    assert set(symbols) == set(_hip.SIGNATURES), "ctypes signatures must cover the header"
    lib = ctypes.CDLL(_hip.LIBRARY_PATH)
    for name in symbols:
        assert hasattr(lib, name), name
    bound = _hip.library()
    assert bound.vrh_abi_version() == _hip.ABI_VERSION
    assert bound.vrh_paged_decode_workspace_bytes(64, 16, 128) >= 64 * 16 * 16 * 130 * 4


def test_prefill_workspace_covers_the_decode_rows_it_routes():
    """A packed batch with max_seqlen_q <= 8 runs every query as a decode row
    (num_seqs x max_seqlen_q rows of split partials); longer batches route only
    their one-query sequences (num_seqs rows). Both also hold the int32
    dispatch order after 256-byte-aligned partials."""
    lib = _hip.library()
    dec = lib.vrh_paged_decode_workspace_bytes
    pre = lib.vrh_paged_prefill_workspace_bytes
    for seqs in (1, 7, 64, 100):
        for max_q in (1, 2, 5, 8):
            need = -(-dec(seqs * max_q, 16, 128) // 256) * 256
            assert pre(seqs, max_q, 16, 128) == need + 4 * seqs
        for max_q in (9, 512, 8192):
            need = -(-dec(seqs, 16, 128) // 256) * 256
            assert pre(seqs, max_q, 16, 128) == need + 4 * seqs


def test_library_rejects_bad_arguments_without_a_gpu():
    lib = _hip.library()
    # rows > 0 with a null workspace fails validation before any launch
    code = lib.vrh_paged_decode(2, 1, 1, 1, 1, 1, 1, 4, 16, 16, 128, 16, 8, 8, 1, 1, 1, 1, 1, 1,
                                1, 1, 1, 1, 0, None, 0, None)
    assert code == 1 and b"workspace" in lib.vrh_last_error()
    code = lib.vrh_kv_append(9, 1, 1, 1, 1, 1, 0, 1, 1, 1, 1, 0, 1, 1, 0, 1, 1, None, None, 1, 1,
                             1, 1, 0, 0, None)
    assert code == 1 and b"dtype" in lib.vrh_last_error()
    code = lib.vrh_kv_finalize_token(1, 1, 0, (ctypes.c_int64 * 1)(0), 1, 0,
                                     (ctypes.c_int32 * 1)(0), 1, 64, 64, 64, 64, None)
    assert code == 1 and b"destination" in lib.vrh_last_error()
    # zero-size work is a no-op success
    assert lib.vrh_kv_copy_blocks(1, 1, 64, 64, 1, 1, 0, None) == 0


def test_silu_and_mul_argument_contract_on_cpu():
    # reference tests/test_activation.py:79-95: checks precede any device work
    from vllm_rlt.kernels.activation import silu_and_mul

    with pytest.raises(ValueError, match="same shape"):
        silu_and_mul(torch.ones(2, 7), torch.ones(1, 7))
    with pytest.raises(TypeError, match="same dtype"):
        silu_and_mul(torch.ones(7), torch.ones(7, dtype=torch.float16))
    for dtype in (torch.int32, torch.float64):
        with pytest.raises(TypeError, match="supports float32"):
            silu_and_mul(torch.ones(7, dtype=dtype), torch.ones(7, dtype=dtype))
    # no CPU path in the hip build
    with pytest.raises(ValueError, match="ROCm"):
        silu_and_mul(torch.ones(7), torch.ones(7))


def test_row_movers_reject_host_tensors_and_bad_shapes():
    from vllm_rlt.kernels import routing

    pool, out = torch.zeros(4, 8), torch.zeros(2, 8)
    with pytest.raises(ValueError, match="ROCm"):
        routing.gather_rows(pool, torch.zeros(2, dtype=torch.int64), out, 2)
    with pytest.raises(ValueError, match="ROCm"):
        routing.gather_segments(pool, torch.zeros(1, 5, dtype=torch.int64), out, 2, 2)


def test_silu_and_mul_abi_rejects_bad_arguments_without_a_gpu():
    lib = _hip.library()
    assert lib.vrh_silu_and_mul(7, 16, 16, 16, 4, None) == 1
    assert b"supports float32" in lib.vrh_last_error()
    assert lib.vrh_silu_and_mul(2, 16, 16, 16, -1, None) == 1
    assert lib.vrh_silu_and_mul(2, 0, 16, 16, 0, None) == 0          # empty: no launch
    assert lib.vrh_silu_and_mul(2, 16, 17, 16, 4, None) == 1         # bf16 pointer misaligned
    assert b"aligned" in lib.vrh_last_error()
    assert lib.vrh_gather_rows(16, 16, 16, 0, 4, 64, 32, 64, None) == 1  # stride < width
    assert b"stride" in lib.vrh_last_error()
