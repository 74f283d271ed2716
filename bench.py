"""Benchmark of the gfx950 paged-KV hot path on one MI355X.

Workload: Ouro-1.4B decode over a LAST_EXITED pool —
64 requests x 4 depth planes, 24 layers, 16 heads x 128, block 16, bf16
N(0,1)*0.5, context ~ U[512, 4096], each row at a random depth plane. A step
is one recurrent traversal: for each of the 24 layers, a paged decode call
over that layer's view of the pool (inputs resident in HBM).

value = algorithmic decode bytes per step / wall time per step, in GB/s
(K+V of every visible token per row + q/out + page-table entries).
Also reported (same JSON line, "extras"): KV-append GB/s for a 24-layer
batched append of the step's tokens and for the config-4 chunk append (8,039
rows), whole-block copy and LAST_EXITED finalize GB/s on the config-2 pool,
config-3 (SHARED, shared prefix pages) decode GB/s, packed prefill TFLOP/s at
config 4; plus the HIP-event roofline of the decode kernel pair and the CPU
oracle baseline on a bounded sample.

    python bench.py [--gpus 1] [--steps 300] [--warmup 10]
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _path in (ROOT, os.path.join(ROOT, "vllm-rlt_amd")):
    if _path not in sys.path:
        sys.path.insert(0, _path)

HBM_PEAK_GBS = 8000.0
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "paged_decode_config2.md")


def profiled_traffic(path=TRAFFIC_PROFILE):
    """HBM bytes per call from a committed rocprof PMC summary (scaled
    FETCH_SIZE + WRITE_SIZE of the call's kernels), or None."""
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_call:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None
BF16_PEAK_TFLOPS = 2500.0


def parse_args():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=300)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--eager", action="store_true",
                        help="time the decode step as eager launches instead of a HIP graph")
    parser.add_argument("--skip-extras", action="store_true",
                        help="only the decode step (no append/prefill/cpu legs)")
    parser.add_argument("--cpu-seconds", type=float, default=10.0,
                        help="budget of the CPU baseline sample")
    parser.add_argument("--leg", choices=["prefill_config4", "prefill_chunks_config4",
                                          "append_config4", "append_config2", "decode_config2",
                                          "decode_config3", "decode_config5", "decode_gqa",
                                          "movers"],
                        help="run only this workload (for profiling) and print its timing")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run vrh_kv_copy_blocks over a known byte count (the "
                             "reference kernel for scaling rocprof FETCH_SIZE/WRITE_SIZE)")
    return parser.parse_args()


def copy_calibration():
    """Copy 512 blocks of 1 MiB each (K and V): 1 GiB read + 1 GiB written per
    launch, 5 launches. Prints the byte counts the counters should report."""
    import torch

    from vllm_rlt.kernels.hip_attention import kv_copy_blocks

    device = torch.device("cuda:0")
    pool_k = torch.zeros((1024, 1 << 19), dtype=torch.bfloat16, device=device)
    pool_v = torch.zeros_like(pool_k)
    src = torch.arange(0, 512, dtype=torch.int64, device=device)
    dst = src + 512
    for _ in range(5):
        kv_copy_blocks(pool_k, pool_v, src, dst)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"read_bytes": 2 * 512 * (1 << 20),
                                           "write_bytes": 2 * 512 * (1 << 20)}}))


def event_time_ms(fn, repeats):
    """Average HIP-event time of ``fn`` on the current stream."""
    import torch

    starts = [torch.cuda.Event(enable_timing=True) for _ in range(repeats)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(repeats)]
    for i in range(repeats):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    return sum(s.elapsed_time(e) for s, e in zip(starts, ends)) / repeats


def graph_time_ms(fns, replays=10):
    """Kernel time per call without Python launch overhead: capture the calls
    ``fns`` (one or a list, run back to back) in one HIP graph, replay it
    ``replays`` times and divide the HIP-event time by the number of calls."""
    import torch

    fns = fns if isinstance(fns, (list, tuple)) else [fns]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for fn in fns:
            fn()  # warm up outside capture (library load, allocator)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for fn in fns:
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (replays * len(fns))


def cpu_baseline(work, budget_s):
    """The reference's decode attention restated in Torch on the host CPU
    (oracle/torch_ref.py, same operations as kernels/paged_attention.py:12-36),
    timed on a bounded sample: whole layers of the config-2 batch, each row's
    pages copied to host memory beforehand, until half of ``budget_s`` per
    thread count. Reported with k host threads (the value) and with 1."""
    import torch

    from oracle import torch_ref

    rows = work.rows
    tables = work.block_tables.cpu()
    lengths = work.context_lengths.cpu()
    es = work.key_cache.element_size()
    hkv, d = work.key_cache.shape[3], work.key_cache.shape[4]
    share = os.environ.get("OMP_NUM_THREADS")
    cores = len(os.sched_getaffinity(0))
    k = min(cores, int(share)) if share and share.isdigit() else cores
    # host copy of one layer's visible pages, compacted, with remapped tables
    samples = []
    for layer in range(work.layers):
        kc, vc = work.key_cache[:, layer], work.value_cache[:, layer]
        pages = [tables[r, : -(-int(lengths[r]) // 16)].to(torch.int64) for r in range(rows)]
        flat = torch.cat(pages)
        local = torch.zeros_like(tables)
        start = 0
        for r, p in enumerate(pages):
            local[r, : len(p)] = torch.arange(start, start + len(p), dtype=torch.int32)
            start += len(p)
        samples.append((kc[flat.to(kc.device)].cpu(), vc[flat.to(vc.device)].cpu(), local))
        if len(samples) >= 1:  # one layer (~1.2 GB of host pages) is reused
            break
    q = work.q.cpu()
    layer_bytes = sum(int(n) * 2 * hkv * d * es + 2 * q[0].numel() * es + -(-int(n) // 16) * 4
                      for n in lengths.tolist())

    def run(threads):
        torch.set_num_threads(threads)
        done, elapsed, layers_done = 0, 0.0, 0
        while elapsed < budget_s / 2:
            kc, vc, local = samples[layers_done % len(samples)]
            t0 = time.perf_counter()
            torch_ref.paged_attention(q, kc, vc, local, lengths)
            elapsed += time.perf_counter() - t0
            done += layer_bytes
            layers_done += 1
        return done / elapsed / 1e9, layers_done, elapsed

    threads_before = torch.get_num_threads()
    single, n1, t1 = run(1)
    multi, nk, tk = run(k)
    torch.set_num_threads(threads_before)
    legs = cpu_legs(k, budget_s / 6)
    return {
        "value": round(multi, 4),
        "unit": "GB/s",
        "cores": k,
        "kind": "port",
        "single_thread_value": round(single, 4),
        "sample": f"Torch-on-CPU restatement of the reference decode (oracle/torch_ref.py) over "
                  f"the {rows} config-2 rows of one layer call, host-resident pages: {nk} layer "
                  f"calls in {tk:.1f} s with {k} threads; {n1} in {t1:.1f} s with 1 thread",
        "legs": legs,
    }


def _timed(fn, budget_s):
    """Repeat ``fn`` until ``budget_s`` seconds have passed; (calls, seconds)."""
    calls, elapsed = 0, 0.0
    while elapsed < budget_s or calls == 0:
        t0 = time.perf_counter()
        fn()
        elapsed += time.perf_counter() - t0
        calls += 1
    return calls, elapsed


def cpu_legs(threads, budget_s):
    """The reference's other host operations on the host CPU, with ``threads``
    Torch threads, each on a bounded sample whose shape is named in its entry:
    config 1 in full, the index-put append (kv_cache_manager.py:698-699) of the
    config-2 step (24 layers x 64 rows) and of a config-4 chunk batch, and
    decode / prefill on row subsamples of configs 3 and 4 built on the host
    with the same generators (fewer groups / prompts)."""
    import torch

    from oracle import torch_ref
    from vllm_rlt import workloads

    threads_before = torch.get_num_threads()
    torch.set_num_threads(threads)
    legs = {}
    try:
        w1 = workloads.config1(device="cpu")
        calls, secs = _timed(lambda: torch_ref.paged_attention(
            w1.q, w1.key_cache[:, 0], w1.value_cache[:, 0], w1.block_tables,
            w1.context_lengths), budget_s)
        legs["decode_config1_full"] = {"gbs": round(w1.decode_bytes() * calls / secs / 1e9, 4),
                                       "calls": calls, "s": round(secs, 2),
                                       "sample": "config 1 in full (8 fp32 rows)"}
        # config-2 step append: the 64 rows' destination pages compacted into a
        # 64-block host pool of the real 24-layer block shape
        w2 = workloads.config2(device="cpu", rows=64, layers=24, fill=False)
        pool_k = torch.zeros((64, 24, 16, 16, 128), dtype=torch.bfloat16)
        pool_v = torch.zeros_like(pool_k)
        blocks = torch.randperm(64, generator=torch.Generator().manual_seed(3))
        offsets = w2.write_offsets

        def append_step():
            for layer in range(24):
                torch_ref.append(pool_k, pool_v, layer, w2.k_new[layer], w2.v_new[layer],
                                 blocks, offsets)

        calls, secs = _timed(append_step, budget_s)
        legs["append_config2_24_layers"] = {
            "gbs": round(w2.append_bytes(24) * calls / secs / 1e9, 4), "calls": calls,
            "s": round(secs, 2), "sample": "config-2 step: 24 layers x 64 rows, index-put"}
        del w2, pool_k, pool_v
        # config 4 subsample: 2 prompts' chunks + 6 decode rows
        w4 = workloads.config4(device="cpu", prompts=2, decode_rows=6)
        pool_k = w4.key_cache.clone()
        pool_v = w4.value_cache.clone()
        calls, secs = _timed(lambda: torch_ref.append(pool_k, pool_v, 0, w4.k_new, w4.v_new,
                                                      w4.write_blocks, w4.write_offsets),
                             budget_s)
        legs["append_config4_subsample"] = {
            "gbs": round(w4.append_bytes() * calls / secs / 1e9, 4), "calls": calls,
            "s": round(secs, 2), "rows": int(w4.k_new.shape[0]),
            "sample": "config-4 shape, 2 prompts' chunks + 6 decode rows, index-put"}
        # prefill: the first 32 queries of each chunk plus the decode rows
        cu = w4.cu_seqlens_q.tolist()
        keep_q, keep_cu, keep_n = [], [0], []
        n = w4.context_lengths.tolist()
        for s in range(len(n)):
            q_len = cu[s + 1] - cu[s]
            take = min(32, q_len)
            keep_q.extend(range(cu[s], cu[s] + take))
            keep_cu.append(keep_cu[-1] + take)
            keep_n.append(n[s] - q_len + take)
        qs = w4.q[keep_q]
        cu_t = torch.tensor(keep_cu, dtype=torch.int32)
        n_t = torch.tensor(keep_n, dtype=torch.int32)
        flops = 4 * 128 * 16 * sum(keep_n[s] - (keep_cu[s + 1] - keep_cu[s]) + i + 1
                                   for s in range(len(keep_n))
                                   for i in range(keep_cu[s + 1] - keep_cu[s]))
        calls, secs = _timed(lambda: torch_ref.prefill(qs, w4.key_cache[:, 0],
                                                       w4.value_cache[:, 0], w4.block_tables,
                                                       n_t, cu_t), budget_s)
        legs["prefill_config4_subsample"] = {
            "gflops": round(flops * calls / secs / 1e9, 3), "calls": calls,
            "s": round(secs, 2), "queries": len(keep_q),
            "sample": "config-4 shape, 2 prompts: first 32 queries of each chunk + 6 decode "
                      "rows, as per-query decode rows"}
        del w4, pool_k, pool_v
        w3 = workloads.config3(device="cpu", groups=2)
        calls, secs = _timed(lambda: torch_ref.paged_attention(
            w3.q, w3.key_cache[:, 0], w3.value_cache[:, 0], w3.block_tables,
            w3.context_lengths), budget_s)
        legs["decode_config3_subsample"] = {
            "gbs": round(w3.decode_bytes() * calls / secs / 1e9, 4), "calls": calls,
            "s": round(secs, 2), "rows": w3.rows,
            "sample": "config-3 shape, 2 groups of 8 rows sharing a 1024-token prefix"}
    finally:
        torch.set_num_threads(threads_before)
    return legs


def mlp_and_rows_extras(device, chunk_rows):
    """SiLU-and-Mul at the Ouro-1.4B MLP width and the WCPB hidden-state segment
    gather/scatter of the config-4 chunks (HBM-bound byte movers)."""
    import torch

    from vllm_rlt.kernels.activation import silu_and_mul
    from vllm_rlt.kernels.routing import gather_segments, scatter_segments

    out = {}
    gen = torch.Generator().manual_seed(1)
    inter = 5632
    for name, tokens, offset in (("silu_and_mul_prefill_8192x5632", 8192, 0),
                                 ("silu_and_mul_prefill_8192x5632_misaligned", 8192, 1),
                                 ("silu_and_mul_decode_64x5632", 64, 0)):
        count = tokens * inter
        gate = torch.randn(count + offset, generator=gen).to(torch.bfloat16).to(device)[offset:]
        up = torch.randn(count + offset, generator=gen).to(torch.bfloat16).to(device)[offset:]
        ms = graph_time_ms([lambda g=gate, u=up: silu_and_mul(g, u)] * 8)
        nbytes = count * 2 * 3
        out[name] = {"gbs": round(nbytes / (ms * 1e-3) / 1e9, 2), "us": round(ms * 1e3, 2),
                     "pct_of_hbm_peak": round(100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)}
        del gate, up
    # Hidden-state segments: 4 disjoint sets of pool rows and batch buffers
    # (268 MB in all), rotated so that no call re-reads the previous ones'.
    hidden = 2048
    slots, pool_rows = 64, 1024
    pool = torch.randn(slots * pool_rows, hidden, generator=gen).to(torch.bfloat16).to(device)
    segment_sets, batches = [], []
    for k in range(4):
        seg = [[(7 * i + 16 * k) % slots, 512 * (i % 2), 512, 512 * i, 1]
               for i in range(chunk_rows // 512)]
        segment_sets.append(torch.tensor(seg, dtype=torch.int64, device=device))
        batches.append(torch.empty(chunk_rows, hidden, dtype=torch.bfloat16, device=device))
    g_ms = graph_time_ms([lambda k=k: gather_segments(pool, segment_sets[k], batches[k], pool_rows,
                                                      512) for k in range(4)] * 4)
    s_ms = graph_time_ms([lambda k=k: scatter_segments(batches[k], segment_sets[k], pool,
                                                       pool_rows, 512) for k in range(4)] * 4)
    nbytes = chunk_rows * hidden * 2 * 2
    for name, ms in (("gather_segments_config4", g_ms), ("scatter_segments_config4", s_ms)):
        out[name] = {"gbs": round(nbytes / (ms * 1e-3) / 1e9, 2), "us": round(ms * 1e3, 2),
                     "rows": chunk_rows}
    return out


def metadata_extras(device):
    """The integer routing / address kernels at decode and WCPB sizes (latency:
    microseconds per call, graph-timed) and the ``read`` gather of one
    4096-token request (bytes read + written)."""
    import torch

    from vllm_rlt.kernels.hip_attention import (
        expand_kv_addresses,
        kv_gather,
        routing_metadata,
        routing_slots,
    )

    gen = torch.Generator().manual_seed(3)
    out = {}
    # async routing of a 64-row decode batch: 64 slots x 4 planes, 257-page tables
    rows, planes, width, page = 64, 4, 257, 16
    tables = torch.randint(0, 40000, (rows * planes, width), generator=gen,
                           dtype=torch.int32).to(device)
    desc = torch.stack([torch.randperm(rows, generator=gen), torch.randint(0, planes, (rows,),
                        generator=gen), torch.randint(0, width * page, (rows,), generator=gen)],
                       1).to(torch.int64).to(device)
    i64 = lambda: torch.empty(rows, dtype=torch.int64, device=device)
    slots, positions, blocks, offsets = i64(), i64(), i64(), i64()
    lengths = torch.empty(rows, dtype=torch.int32, device=device)
    out_tables = torch.empty((rows, width), dtype=torch.int32, device=device)
    meta_ms = graph_time_ms([lambda: routing_metadata(
        desc, tables, n=rows, size=rows, width=width, page=page, planes=planes,
        out_width=width, slots=slots, positions=positions, lengths=lengths, blocks=blocks,
        offsets=offsets, out_tables=out_tables)] * 32)
    slots_ms = graph_time_ms([lambda: routing_slots(desc, slots, rows, rows)] * 32)
    # WCPB write addresses of the config-4 batch size
    n = 8039
    pos = torch.randint(0, 8192, (n,), generator=gen, dtype=torch.int64).to(device)
    seqs = torch.randint(0, 64, (n,), generator=gen, dtype=torch.int32).to(device)
    tab = torch.randint(0, 40000, (64, 513), generator=gen, dtype=torch.int32).to(device)
    b8, o8 = torch.empty(n, dtype=torch.int64, device=device), torch.empty(n, dtype=torch.int64,
                                                                            device=device)
    expand_ms = graph_time_ms([lambda: expand_kv_addresses(pos, seqs, tab, 16, b8, o8)] * 32)
    out["routing_metadata_64_rows_us"] = round(meta_ms * 1e3, 2)
    out["routing_slots_64_rows_us"] = round(slots_ms * 1e3, 2)
    out["expand_kv_addresses_8039_us"] = round(expand_ms * 1e3, 2)
    # read (kv_gather) of a 4096-token request from a 24-layer pool layer
    # view, rotating over 4 requests with disjoint pages
    pool = torch.empty((1100, 24, 16, 16, 128), dtype=torch.bfloat16, device=device).normal_()
    tables = torch.randperm(1100, generator=gen)[:1024].to(torch.int32).to(device).view(4, 256)
    kview, vview = pool[:, 5], pool[:, 7]
    gather_ms = graph_time_ms([lambda k=k: kv_gather(kview, vview, tables[k], 4096)
                               for k in range(4)] * 2)
    gbytes = 4096 * 16 * 128 * 2 * 2 * 2
    out["kv_gather_4096_tokens"] = {"gbs": round(gbytes / (gather_ms * 1e-3) / 1e9, 2),
                                    "us": round(gather_ms * 1e3, 2)}
    return out


def offload_extras(device):
    """Preemption snapshot/restore of a 4096-token Ouro-1.4B request (256 pages of
    3 MiB, K + V) through pinned host memory: one launch per direction, against
    the reference's one copy per page. Host-link bound (PCIe 5.0 x16: 64 GB/s)."""
    import torch

    from vllm_rlt.kernels.hip_attention import kv_blocks_from_host, kv_blocks_to_host

    pages = 256
    shape = (pages + 64, 24, 16, 16, 128)
    key_pool = torch.randn(shape[1:], dtype=torch.bfloat16, device=device).expand(shape).clone()
    value_pool = key_pool.clone()
    blocks = torch.randperm(pages + 64)[:pages]
    index = blocks.to(device)
    host_k = torch.empty((pages, *shape[1:]), dtype=torch.bfloat16, pin_memory=True)
    host_v = torch.empty_like(host_k, pin_memory=True)
    nbytes = 2 * host_k.numel() * 2
    kv_blocks_to_host(key_pool, value_pool, index, host_k, host_v)
    torch.cuda.synchronize()
    to_ms = event_time_ms(lambda: kv_blocks_to_host(key_pool, value_pool, index, host_k, host_v), 3)
    from_ms = event_time_ms(
        lambda: kv_blocks_from_host(key_pool, value_pool, index, host_k, host_v), 3)

    def per_page():
        for row, block in enumerate(blocks.tolist()):
            host_k[row].copy_(key_pool[block], non_blocking=True)
            host_v[row].copy_(value_pool[block], non_blocking=True)

    per_page()
    torch.cuda.synchronize()
    page_ms = event_time_ms(per_page, 2)
    return {"snapshot_256_pages_batched": {"gbs": round(nbytes / (to_ms * 1e-3) / 1e9, 2),
                                           "ms": round(to_ms, 3), "bytes": nbytes},
            "restore_256_pages_batched": {"gbs": round(nbytes / (from_ms * 1e-3) / 1e9, 2),
                                          "ms": round(from_ms, 3)},
            "snapshot_256_pages_per_page_copies": {
                "gbs": round(nbytes / (page_ms * 1e-3) / 1e9, 2), "ms": round(page_ms, 3)}}


def rotating_append_config4(pw, sets=8):
    """The config-4 append (every chunk and decode row) over ``sets`` disjoint
    input / destination sets: set s writes its own K/V rows into block
    ``wb + s * N`` of a pool of ``sets * N`` blocks (N = config-4 pool), so
    consecutive calls share neither source nor destination bytes and the
    total (> 1 GB) exceeds the 256 MB last-level cache. Returns the launch
    closures and the bytes of one call."""
    import torch

    from vllm_rlt.kernels.hip_attention import kv_append

    n = pw.key_cache.shape[0]
    shape = (sets * n, *pw.key_cache.shape[1:])
    pool_k = torch.empty(shape, dtype=pw.key_cache.dtype, device=pw.key_cache.device)
    pool_v = torch.empty_like(pool_k)
    rows = pw.k_new.shape[0]
    gen = torch.Generator(device=pool_k.device).manual_seed(17)
    k_sets = torch.randn((sets, *pw.k_new.shape), generator=gen, device=pool_k.device,
                         dtype=torch.float32).to(pw.k_new.dtype)
    v_sets = torch.randn_like(k_sets)
    blocks = [pw.write_blocks + s * n for s in range(sets)]
    kc, vc = pool_k[:, 0], pool_v[:, 0]
    fns = [lambda s=s: kv_append(kc, vc, k_sets[s], v_sets[s], blocks[s], pw.write_offsets)
           for s in range(sets)]
    return fns, pw.append_bytes(), (pool_k, pool_v, k_sets, v_sets), rows


def rotating_append_layers(work, sets=48):
    """The config-2 step append of all 24 layers in one launch, over ``sets``
    disjoint destination slot sets and input sets (25 MB per call, 1.2 GB in
    all), so no call is served from cache."""
    import torch

    from vllm_rlt.kernels.hip_attention import kv_append_layers

    device = work.key_cache.device
    rows = work.rows
    gen = torch.Generator().manual_seed(19)
    slots = torch.randperm(work.num_blocks * 16, generator=gen)[: sets * rows].view(sets, rows)
    blocks = (slots // 16).to(device)
    offsets = (slots % 16).to(device)
    dgen = torch.Generator(device=device).manual_seed(23)
    k_sets = torch.randn((sets, *work.k_new.shape), generator=dgen, device=device,
                         dtype=torch.float32).to(work.k_new.dtype)
    v_sets = torch.randn_like(k_sets)
    fns = [lambda s=s: kv_append_layers(work.key_cache, work.value_cache, 0, k_sets[s],
                                        v_sets[s], blocks[s], offsets[s]) for s in range(sets)]
    return fns, work.append_bytes(work.layers), (k_sets, v_sets, blocks, offsets)


def plain_copy_floor(nbytes_moved, device, sets=48):
    """Graph-timed ``dst.copy_(src)`` of contiguous tensors moving the same
    bytes (half read, half written) over ``sets`` rotating pairs: the time any
    kernel needs to move that many bytes in one launch on this chip."""
    import torch

    elems = nbytes_moved // 2 // 2  # bf16 elements read (= written)
    src = [torch.empty(elems, dtype=torch.bfloat16, device=device).normal_()
           for _ in range(sets)]
    dst = [torch.empty_like(x) for x in src]
    ms = graph_time_ms([lambda i=i: dst[i].copy_(src[i]) for i in range(sets)], replays=2)
    del src, dst
    return ms


def decode_config5_leg(device, calls=6):
    """Config 5's decode shape: 256 rows, context U[2048, 32768], over one layer
    view of a 48-layer pool of 32768 blocks (6 MiB of K+V per block: 192 GiB,
    the ~200 GB pool of the configuration) with 2048-page tables."""
    import torch

    from vllm_rlt import workloads
    from vllm_rlt.kernels.hip_attention import paged_attention

    w = workloads.config5(device=device)
    layer = 24
    kc, vc = w.key_cache[:, layer], w.value_cache[:, layer]
    call = lambda: paged_attention(w.q, kc, vc, w.block_tables, w.context_lengths)  # noqa: E731
    ms = graph_time_ms([call] * calls, replays=2)
    nbytes = w.decode_bytes()
    tokens = int(w.context_lengths.sum())
    slots = w.num_blocks * w.key_cache.shape[2]
    out = {"gbs": round(nbytes / (ms * 1e-3) / 1e9, 2), "ms": round(ms, 4),
           "pct_of_hbm_peak": round(100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
           "bytes_per_call": nbytes, "rows": w.rows, "pool_blocks": w.num_blocks,
           "tokens": tokens, "page_reuse": round(tokens / slots, 2),
           "bytes": "gbs counts K/V once per row that reads it (rows share random pages, "
                    f"{tokens} tokens over {slots} slots)"}
    traffic = profiled_traffic(os.path.join(ROOT, "profiles", "paged_decode_config5.md"))
    if traffic:
        # HBM bytes per call measured by FETCH_SIZE / WRITE_SIZE (scaled by a
        # calibration copy): the rate on bytes the memory actually delivered.
        out["traffic_bytes_per_call"] = traffic
        out["gbs_counter_bytes"] = round(traffic / (ms * 1e-3) / 1e9, 2)
        out["pct_of_hbm_peak_counter_bytes"] = round(
            100 * traffic / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)
    del w, kc, vc
    torch.cuda.empty_cache()
    return out


def decode_gqa_leg(device, calls=8, q_heads=32, kv_heads=8):
    """Grouped-query decode: config 2's 64 rows and context range with q_heads
    q heads over kv_heads kv heads (head_dim 128, bf16). Algorithmic bytes
    count each K/V byte once per row (what one wave per kv head reads). Groups
    of 4 run on the VALU kernel, groups of 8 on the MFMA kernel."""
    import torch

    from vllm_rlt import workloads
    from vllm_rlt.kernels.hip_attention import paged_attention

    w = workloads.gqa_decode(device=device, q_heads=q_heads, kv_heads=kv_heads)
    kc, vc = w.key_cache[:, 0], w.value_cache[:, 0]
    call = lambda: paged_attention(w.q, kc, vc, w.block_tables, w.context_lengths)  # noqa: E731
    ms = graph_time_ms([call] * calls, replays=4)
    nbytes = w.decode_bytes()
    out = {"gbs": round(nbytes / (ms * 1e-3) / 1e9, 2), "us": round(ms * 1e3, 2),
           "pct_of_hbm_peak": round(100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
           "bytes_per_call": nbytes, "rows": w.rows, "q_heads": q_heads, "kv_heads": kv_heads}
    del w, kc, vc
    torch.cuda.empty_cache()
    return out


def pool_movers(work, replays=2):
    """Whole-block copy and LAST_EXITED finalize on the config-2 pool, each over
    16 disjoint sets so that no call re-reads bytes a previous one touched.
    copy: 64 random 3 MiB blocks (K and V) per call; finalize: the 64 rows'
    tokens at 16 different positions, from their depth plane into every
    deeper plane, all 24 layers."""
    import torch

    from vllm_rlt.kernels.hip_attention import kv_copy_blocks, kv_finalize

    device = work.key_cache.device
    layers = work.layers
    gen = torch.Generator().manual_seed(5)
    perm = torch.randperm(work.num_blocks, generator=gen)[: 128 * 16].to(device).view(16, 128)
    copy_ms = graph_time_ms(
        [lambda i=i: kv_copy_blocks(work.key_cache, work.value_cache, perm[i, :64],
                                    perm[i, 64:]) for i in range(16)], replays=replays)
    block_bytes = work.key_cache[0].numel() * work.key_cache.element_size()
    copy_bytes = 64 * block_bytes * 2 * 2
    depths = work.extra["depths"]
    planes = 4
    plane_tables = work.extra["plane_tables"]
    width = max(len(t) for t in plane_tables)
    table_dev = torch.zeros((len(plane_tables), width), dtype=torch.int32)
    for i, pages in enumerate(plane_tables):
        table_dev[i, : len(pages)] = torch.tensor(pages, dtype=torch.int32)
    table_dev = table_dev.to(device)
    last = (work.context_lengths - 1).to(torch.int64).cpu()
    descs = [torch.stack([torch.arange(work.rows), depths.to(torch.int64), last - k], 1).to(device)
             for k in range(16)]
    fin_ms = graph_time_ms(
        [lambda d=d: kv_finalize(work.key_cache, work.value_cache, d, table_dev, planes)
         for d in descs], replays=replays)
    slot = work.key_cache.shape[3] * work.key_cache.shape[4] * work.key_cache.element_size()
    fin_bytes = int((planes - 1 - depths).sum()) * layers * slot * 2 * 2
    return {"copy_blocks_64x3MiB": {"gbs": round(copy_bytes / (copy_ms * 1e-3) / 1e9, 2),
                                    "us": round(copy_ms * 1e3, 2), "bytes": copy_bytes},
            "finalize_64_tokens_24_layers": {"gbs": round(fin_bytes / (fin_ms * 1e-3) / 1e9, 2),
                                             "us": round(fin_ms * 1e3, 2), "bytes": fin_bytes,
                                             "rotation": "16 token positions per row"}}


def single_leg(name, repeats):
    """One workload alone, for rocprofv3 runs (kernel durations and counters of
    that workload only)."""
    import torch

    from vllm_rlt import workloads
    from vllm_rlt.kernels.hip_attention import paged_attention, paged_prefill_attention

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if name in ("prefill_config4", "prefill_chunks_config4"):
        kw = {"decode_rows": 0} if name == "prefill_chunks_config4" else {}
        pw = workloads.config4(device=device, **kw)
        kc, vc = pw.key_cache[:, 0], pw.value_cache[:, 0]
        ms = event_time_ms(lambda: paged_prefill_attention(pw.q, kc, vc, pw.block_tables,
                                                           pw.context_lengths, pw.cu_seqlens_q,
                                                           pw.max_seqlen_q), repeats)
        flops = pw.flops()
        print(json.dumps({"leg": name, "ms": round(ms, 4),
                          "tflops": round(flops / (ms * 1e-3) / 1e12, 2), "flops": flops}),
              flush=True)
    elif name == "append_config4":
        pw = workloads.config4(device=device)
        fns, nbytes, _keep, rows = rotating_append_config4(pw)
        ms = event_time_ms(lambda: [fn() for fn in fns], repeats) / len(fns)
        print(json.dumps({"leg": name, "us": round(ms * 1e3, 2), "bytes_per_call": nbytes,
                          "rows": rows, "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2)}),
              flush=True)
    elif name == "append_config2":
        w = workloads.config2(device=device)
        fns, nbytes, _keep = rotating_append_layers(w)
        ms = event_time_ms(lambda: [fn() for fn in fns], repeats) / len(fns)
        print(json.dumps({"leg": name, "us": round(ms * 1e3, 2), "bytes_per_call": nbytes,
                          "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2)}), flush=True)
    elif name == "decode_config2":
        w = workloads.config2(device=device)
        layers = [(w.key_cache[:, l], w.value_cache[:, l]) for l in range(w.layers)]
        ms = event_time_ms(lambda: [paged_attention(w.q, k, v, w.block_tables,
                                                    w.context_lengths) for k, v in layers],
                           repeats) / w.layers
        nbytes = w.decode_bytes()
        print(json.dumps({"leg": name, "us": round(ms * 1e3, 2), "bytes_per_call": nbytes,
                          "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2)}), flush=True)
    elif name == "movers":
        # every byte mover of the path once per replay, for counter runs
        w = workloads.config2(device=device)
        out = pool_movers(w, replays=repeats)
        del w
        torch.cuda.empty_cache()
        out.update(mlp_and_rows_extras(device, 8192))
        out.update(metadata_extras(device))
        print(json.dumps({"leg": name, **out}), flush=True)
    elif name == "decode_gqa":
        print(json.dumps({"leg": name, **decode_gqa_leg(device, calls=repeats)}), flush=True)
        print(json.dumps({"leg": name, **decode_gqa_leg(device, calls=repeats, q_heads=64)}),
              flush=True)
    elif name == "decode_config5":
        print(json.dumps({"leg": name, **decode_config5_leg(device, calls=repeats)}),
              flush=True)
    elif name == "decode_config3":
        w = workloads.config3(device=device)
        k, v = w.key_cache[:, 0], w.value_cache[:, 0]
        ms = event_time_ms(lambda: paged_attention(w.q, k, v, w.block_tables,
                                                   w.context_lengths), repeats)
        es = w.key_cache.element_size()
        unique = w.extra["unique_tokens"] * 2 * w.key_cache.shape[3] * w.key_cache.shape[4] * es
        print(json.dumps({"leg": name, "us": round(ms * 1e3, 2), "per_row_bytes": w.decode_bytes(),
                          "unique_kv_bytes": unique}), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}); this build has no "
              "multi-GPU path", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        copy_calibration()
        return
    if args.leg:
        single_leg(args.leg, args.steps)
        return
    import torch

    from vllm_rlt import workloads
    from vllm_rlt.kernels._extension import load_extension
    from vllm_rlt.kernels._hip import library
    from vllm_rlt.kernels.hip_attention import (
        kv_append,
        kv_append_layers,
        paged_attention,
        paged_prefill_attention,
    )

    library()
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    work = workloads.config2(device=device)
    layers = work.layers
    kviews = [work.key_cache[:, layer] for layer in range(layers)]
    vviews = [work.value_cache[:, layer] for layer in range(layers)]
    tables, lengths, q = work.block_tables, work.context_lengths, work.q

    def eager_step():
        for layer in range(layers):
            paged_attention(q, kviews[layer], vviews[layer], tables, lengths)

    # The reference runs decode steps under CUDA graphs (worker/cuda_graph.py);
    # one step = one replay of the 24 captured layer calls (same kernels and
    # bytes as the eager loop, without per-launch host gaps). --eager times
    # the eager loop instead.
    step = eager_step
    if not args.eager:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            eager_step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            eager_step()
        step = graph.replay

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start_ev = torch.cuda.Event(enable_timing=True)
    end_ev = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start_ev.record()
    for _ in range(args.steps):
        step()
    end_ev.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # HIP-event time of the timed region on the stream the kernels run on;
    # one decode call = split kernel + merge kernel.
    call_ms = start_ev.elapsed_time(end_ev) / (args.steps * layers)
    ms_per_step = wall * 1e3 / args.steps
    decode_bytes = work.decode_bytes()
    step_bytes = decode_bytes * layers
    value = step_bytes / (wall / args.steps) / 1e9

    achieved = decode_bytes / (call_ms * 1e-3) / 1e9
    result = {
        "metric": "paged-decode KV GB/s (% of HBM peak) + KV-append GB/s, Ouro-1.4B shape",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "config2: Ouro-1.4B LAST_EXITED decode, 64 rows x 24 layers, "
                        "16x128 MHA, block 16, ctx U[512,4096], 4 depth planes",
            "rows": work.rows,
            "layers": layers,
            "pool_blocks": work.num_blocks,
            "decode_bytes_per_layer_call": decode_bytes,
            "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "tokens_per_s": round(work.rows * layers / (wall / args.steps), 1),
            "step": "eager launches" if args.eager else "HIP graph replay of the 24 layer calls",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(),
            "kernel": "paged_decode_kernel<bf16,8,16> + paged_decode_merge_kernel<bf16,2> "
                      "(one decode call)",
            "call_ms": round(call_ms, 5),
        },
    }

    if not args.skip_extras:
        # Eager step: the 24 layer calls launched from Python through the
        # ctypes boundary (host argument marshalling included), for comparison
        # with the graph-replayed step above.
        eager_ms = event_time_ms(eager_step, 20)
        # The same step through the registered torch op (vllm_rlt._C), and the
        # host time per call of each boundary (submission only: the GPU runs
        # behind, so the host loop measures argument checks and marshalling).
        load_extension()
        decode_op = torch.ops.vllm_rlt_hip.paged_attention

        def eager_op_step():
            for layer in range(layers):
                decode_op(q, kviews[layer], vviews[layer], tables, lengths, 0)

        eager_op_ms = event_time_ms(eager_op_step, 20)
        host_us = {}
        for name, fn in (("ctypes", eager_step), ("torch_op", eager_op_step)):
            torch.cuda.synchronize()
            t_host = time.perf_counter()
            for _ in range(4):
                fn()
            host_us[name] = round((time.perf_counter() - t_host) * 1e6 / (4 * layers), 2)
            torch.cuda.synchronize()
        # 24-layer batched append of the step's 64 tokens (one launch), over
        # 48 disjoint input / destination sets (1.2 GB in all).
        fns, append_layers_bytes, keep = rotating_append_layers(work)
        append_layers_ms = graph_time_ms(fns, replays=2)
        del keep, fns
        copy_floor_ms = plain_copy_floor(append_layers_bytes, device)
        # single-layer decode append (latency)
        single_ms = graph_time_ms(
            [lambda layer=layer: kv_append(kviews[layer], vviews[layer], work.k_new[layer],
                                           work.v_new[layer], work.write_blocks,
                                           work.write_offsets) for layer in range(layers)])
        extras = {
            "decode_step_eager_ms": round(eager_ms, 4),
            "decode_step_eager_gbs": round(step_bytes / (eager_ms * 1e-3) / 1e9, 2),
            "decode_step_eager_torch_op_ms": round(eager_op_ms, 4),
            "decode_call_host_us": host_us,
            "append_24_layers": {
                "gbs": round(append_layers_bytes / (append_layers_ms * 1e-3) / 1e9, 2),
                "us": round(append_layers_ms * 1e3, 2), "bytes": append_layers_bytes,
                "pct_of_hbm_peak": round(100 * append_layers_bytes / (append_layers_ms * 1e-3)
                                         / 1e9 / HBM_PEAK_GBS, 2),
                "rotation": "48 disjoint input/destination sets, 1.2 GB",
                "plain_copy_same_bytes_us": round(copy_floor_ms * 1e3, 2),
                "vs_plain_copy": round(copy_floor_ms / append_layers_ms, 3),
                "plain_copy": "torch copy_ of contiguous tensors moving the same bytes, "
                              "48 rotating pairs, graph-timed"},
            "append_one_layer_us": round(single_ms * 1e3, 2),
            "append_one_layer_gbs": round(work.append_bytes(1) / (single_ms * 1e-3) / 1e9, 2)}
        extras.update(pool_movers(work))
        result["cpu_baseline"] = cpu_baseline(work, args.cpu_seconds)
        del work, kviews, vviews
        torch.cuda.empty_cache()
        # config 3: SHARED layout, 16 groups x 8 requests sharing 64 prefix pages.
        w3 = workloads.config3(device=device)
        k3, v3 = w3.key_cache[:, 0], w3.value_cache[:, 0]
        dec3_ms = graph_time_ms(
            [lambda: paged_attention(w3.q, k3, v3, w3.block_tables, w3.context_lengths)] * 4,
            replays=5)
        es = w3.key_cache.element_size()
        unique = w3.extra["unique_tokens"] * 2 * w3.key_cache.shape[3] * w3.key_cache.shape[4] * es
        extras["decode_config3_shared_prefix"] = {
            "gbs_per_row_bytes": round(w3.decode_bytes() / (dec3_ms * 1e-3) / 1e9, 2),
            "gbs_unique_bytes": round(unique / (dec3_ms * 1e-3) / 1e9, 2),
            "us": round(dec3_ms * 1e3, 2), "rows": w3.rows, "timing": "graph replay, 4 calls x 5"}
        del w3, k3, v3
        torch.cuda.empty_cache()
        print(f"bench: {torch.cuda.memory_allocated() / 2**30:.1f} GiB held before the "
              "192 GiB config-5 pool", file=sys.stderr, flush=True)
        extras["decode_config5_long_context"] = decode_config5_leg(device)
        extras["decode_gqa_32q_8kv"] = decode_gqa_leg(device)
        extras["decode_gqa_64q_8kv"] = decode_gqa_leg(device, q_heads=64)
        pw = workloads.config4(device=device)
        kc, vc = pw.key_cache[:, 0], pw.value_cache[:, 0]
        fns, append_bytes, keep, append_rows = rotating_append_config4(pw)
        append_ms = graph_time_ms(fns, replays=4)
        del fns, keep
        torch.cuda.empty_cache()
        prefill_ms = event_time_ms(
            lambda: paged_prefill_attention(pw.q, kc, vc, pw.block_tables, pw.context_lengths,
                                            pw.cu_seqlens_q, pw.max_seqlen_q), 10)
        flops = pw.flops()
        extras["append_config4_chunks"] = {
            "gbs": round(append_bytes / (append_ms * 1e-3) / 1e9, 2),
            "us": round(append_ms * 1e3, 2), "rows": append_rows, "bytes": append_bytes,
            "pct_of_hbm_peak": round(100 * append_bytes / (append_ms * 1e-3) / 1e9
                                     / HBM_PEAK_GBS, 2),
            "rotation": "8 disjoint input/destination sets, 1.05 GB"}
        prefill_graph_ms = graph_time_ms(
            [lambda: paged_prefill_attention(pw.q, kc, vc, pw.block_tables, pw.context_lengths,
                                             pw.cu_seqlens_q, pw.max_seqlen_q)] * 4, replays=3)
        # Whole packed call: the 16 MFMA chunks plus the 48 decode rows, which
        # run through the HBM-bound split-KV kernel (0.86 GB of K/V).
        # The call mixes MFMA work (the chunks) and HBM work (the decode rows'
        # K/V): its roofline time is the sum of the two at their peaks.
        cu, lens = pw.cu_seqlens_q.tolist(), pw.context_lengths.tolist()
        heads, dim = pw.q.shape[1], pw.q.shape[2]
        kv_heads, elt = pw.key_cache.shape[3], pw.key_cache.element_size()
        chunk_flops = decode_row_bytes = 0
        for s_, n_ in enumerate(lens):
            q_len = cu[s_ + 1] - cu[s_]
            if q_len > 1:
                chunk_flops += 4 * dim * heads * sum(n_ - q_len + i + 1 for i in range(q_len))
            else:
                decode_row_bytes += n_ * 2 * kv_heads * dim * elt + 2 * heads * dim * elt
        roofline_us = (chunk_flops / (BF16_PEAK_TFLOPS * 1e12)
                       + decode_row_bytes / (HBM_PEAK_GBS * 1e9)) * 1e6
        extras["prefill_config4"] = {
            "tflops": round(flops / (prefill_ms * 1e-3) / 1e12, 2), "ms": round(prefill_ms, 4),
            "pct_of_bf16_mfma_peak": round(100 * flops / (prefill_ms * 1e-3) / 1e12
                                           / BF16_PEAK_TFLOPS, 2),
            "graph_ms": round(prefill_graph_ms, 4),
            "graph_tflops": round(flops / (prefill_graph_ms * 1e-3) / 1e12, 2),
            "chunk_flops": chunk_flops, "decode_row_bytes": decode_row_bytes,
            "roofline_us": round(roofline_us, 1),
            "roofline_frac_graph": round(roofline_us / (prefill_graph_ms * 1e3), 4),
            "includes": "16 chunks (MFMA kernel) + 48 decode rows (split-KV decode kernel); "
                        "roofline_us = chunk FLOPs at the bf16 MFMA peak + decode-row bytes at "
                        "the HBM peak"}
        # The 16 chunks alone: the MFMA kernel (sequences ranked in-kernel) and
        # the empty decode-row launch, graph-timed.
        del pw, kc, vc
        torch.cuda.empty_cache()
        pw = workloads.config4(device=device, decode_rows=0)
        kc, vc = pw.key_cache[:, 0], pw.value_cache[:, 0]
        chunks_ms = graph_time_ms(
            [lambda: paged_prefill_attention(pw.q, kc, vc, pw.block_tables, pw.context_lengths,
                                             pw.cu_seqlens_q, pw.max_seqlen_q)] * 4, replays=3)
        chunk_flops = pw.flops()
        # The same chunks through the C ABI without a workspace (a caller that
        # knows its batch has no one-query sequences): no decode-row launch,
        # so the call is the MFMA kernel alone.
        lib = library()
        out_nows = torch.empty_like(pw.q)

        def chunks_no_workspace():
            lib.check(lib.vrh_paged_prefill(
                2, out_nows.data_ptr(), pw.q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                pw.block_tables.data_ptr(), pw.context_lengths.data_ptr(),
                pw.cu_seqlens_q.data_ptr(), pw.block_tables.shape[0], pw.q.shape[0],
                int(pw.max_seqlen_q), pw.q.shape[1], kc.shape[2], pw.q.shape[2], kc.shape[1],
                pw.block_tables.shape[1], pw.block_tables.stride(0), pw.q.stride(0),
                pw.q.stride(1), out_nows.stride(0), out_nows.stride(1), *kc.stride()[:3],
                *vc.stride()[:3], None, 0, torch.cuda.current_stream().cuda_stream),
                "vrh_paged_prefill")

        kernel_ms = graph_time_ms([chunks_no_workspace] * 4, replays=3)
        extras["prefill_config4_chunks_mfma"] = {
            "graph_ms": round(chunks_ms, 4),
            "tflops": round(chunk_flops / (chunks_ms * 1e-3) / 1e12, 2),
            "pct_of_bf16_mfma_peak": round(100 * chunk_flops / (chunks_ms * 1e-3) / 1e12
                                           / BF16_PEAK_TFLOPS, 2),
            "flops": chunk_flops,
            "kernel_only_graph_ms": round(kernel_ms, 4),
            "kernel_only_pct_of_bf16_mfma_peak": round(
                100 * chunk_flops / (kernel_ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 2),
            "kernel_only": "same chunks through vrh_paged_prefill with no workspace: the "
                           "MFMA kernel alone (no decode-row launch and merge)"}
        # Hidden-state segments of the config-4 chunks around prefill: gather the
        # 16 x 512 chunk rows (Ouro hidden 2048, bf16) from the state pool.
        chunk_rows = pw.chunk_sequences * 512
        del pw, kc, vc
        torch.cuda.empty_cache()
        extras.update(mlp_and_rows_extras(device, chunk_rows))
        extras.update(metadata_extras(device))
        extras.update(offload_extras(device))
        result["extras"] = extras
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
