// Paged single-query (decode) attention, split-KV, for gfx950.
//
// Reference semantics: kernels/paged_attention.py:12-71 (torch_paged_attention
// and the windowed variant): per row, keys/values gathered through the row's
// own block table, GQA head h reads kv head h / G, scores scaled by 1/sqrt(D),
// fp32 softmax, output rounded to the storage dtype, zero rows for length 0.
//
// Design (bandwidth-bound; every K/V byte is read once per row and kv head
// for groups of up to 16 q heads):
//  * One 64-lane wavefront per (split, group of HPW q heads, row): HPW = 8, 4
//    or 2 grouped-query heads when they divide the group (each loaded K/V
//    vector serves all of them), else 1. Groups of 8-16 heads, and of 3, 5, 6
//    or 7, run on the MFMA kernel below instead (one wave per kv head). A split is a run of whole
//    pages: bps = max(min_bps, ceil(pages / kMaxSplits)) pages (at least 128
//    tokens, at most 16 splits per row), so the partition depends only on
//    the row's own length -> batch invariance. The split index is rotated
//    per (row, head) so that every XCD receives the same share of splits.
//  * Lane layout: LPT lanes cover one token's head_dim with VEC elements each
//    (16-byte global loads for bf16 D=128: LPT=16), so one wave-wide load
//    instruction fetches TPL = 64 / LPT tokens; U loads of K and U of V are
//    issued back to back per chunk (branch-free: positions past the end
//    re-read the last valid token and are masked).
//  * The row's page ids for up to 64 pages sit in one VGPR (one per lane) and
//    are fetched with ds_bpermute, so the page table is read once per split.
//    Pages shared with a neighbouring row of the batch are read with ordinary
//    (cache-allocating) loads, the others with non-temporal loads.
//  * Each token group keeps its own online-softmax state (m, l, acc) in the
//    log2 domain; groups are merged once per split with cross-lane shuffles,
//    so the inner loop has no cross-row reductions. QK^T partial sums reduce
//    within a 16-lane row with DPP.
//  * Splits of multi-split rows write (m, l, acc) partials to the workspace;
//    a merge kernel combines them in split order (log-sum-exp). Single-split
//    rows write the output directly.
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace vrh {
namespace {

// Wave loads per chunk (in flight per lane for each of K and V), minimum and
// maximum split length, grouped-query heads one wave may serve.
constexpr int kMaxSplits = 16;
constexpr int kSplitTokens = 128;  // minimum tokens per split (whole pages)
constexpr int kMaxHpw = 8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

constexpr int kU = 8;                // wave loads per chunk (K and V each)

template <typename T, int VEC>
__device__ __forceinline__ typename Vec<T, VEC>::raw_t load_kv(const T* p) {
  return load_raw_stream<T, VEC>(p);
}

struct DecodeArgs {
  void* out;
  const void* q;
  const void* k;
  const void* v;
  const int32_t* tables;
  const int32_t* lengths;
  float* part_ml;   // [rows, q_heads, kMaxSplits, 2]
  float* part_acc;  // [rows, q_heads, kMaxSplits, head_dim]
  int64_t q_row, q_head, o_row, o_head;
  int64_t k_block, k_token, k_head;
  int64_t v_block, v_token, v_head;
  int64_t table_stride;
  int64_t row_base;
  int64_t rows;      // rows of the whole call (the launch may cover a chunk)
  // A head's row of K or V is not a whole number of 128-byte cache lines, so
  // neighbouring heads (other waves) share lines: every page is then read
  // with cache-allocating loads.
  int32_t line_shared;
  // Packed-prefill expansion (null for decode): row r is query i of sequence
  // s with cu_q[s] <= r < cu_q[s+1]; it reads table row s with causal length
  // lengths[s] - q_len(s) + i + 1.
  // expand_e > 0: row r is query r % E of sequence r / E, and only sequences
  // with q_len <= E are processed here (the others belong to the MFMA kernel).
  const int32_t* cu_q;
  int32_t num_seqs;
  int32_t expand_e;
  int32_t q_heads, group, head_dim, block_size, bs_shift, window, min_bps, table_width;
  float scale_log2;
};

struct Partition {
  int start;    // first visible token
  int first;    // first page
  int pages;    // pages touched
  int bps;      // pages per split
  int nsplit;
};

__device__ __forceinline__ Partition partition(int n, const DecodeArgs& a) {
  Partition p;
  p.start = (a.window > 0 && n > a.window) ? n - a.window : 0;
  if (a.bs_shift >= 0) {
    p.first = p.start >> a.bs_shift;
    p.pages = ((n + a.block_size - 1) >> a.bs_shift) - p.first;
  } else {
    p.first = p.start / a.block_size;
    p.pages = (n + a.block_size - 1) / a.block_size - p.first;
  }
  p.bps = max(a.min_bps, ceil_div(p.pages, kMaxSplits));
  p.nsplit = ceil_div(p.pages, p.bps);
  return p;
}

__device__ __forceinline__ int clamp_length(int n, const DecodeArgs& a) {
  // A length beyond the table would read past the row's page ids.
  const int64_t cap = (int64_t)a.table_width * a.block_size;
  if (n < 0) return 0;
  return (int64_t)n > cap ? (int)cap : n;
}

// Visible length, table row and query/output row of work row `row`
// (decode: itself); -1 when the row is not handled by this launch.
__device__ __forceinline__ int row_length(int64_t row, const DecodeArgs& a, int64_t* table_row,
                                          int64_t* query_row) {
  if (a.cu_q == nullptr) {
    *table_row = row;
    *query_row = row;
    return clamp_length(a.lengths[row], a);
  }
  int seq, i;
  if (a.expand_e > 0) {
    seq = (int)(row / a.expand_e);
    i = (int)(row - (int64_t)seq * a.expand_e);
  } else {
    // Rows outside [cu_q[0], cu_q[num_seqs]) (padding of a bucketed q) belong
    // to no sequence.
    if (row < a.cu_q[0] || row >= a.cu_q[a.num_seqs]) return -1;
    int lo = 0, hi = a.num_seqs - 1;  // last s with cu_q[s] <= row
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (a.cu_q[mid] <= row) lo = mid; else hi = mid - 1;
    }
    seq = lo;
    i = (int)(row - a.cu_q[lo]);
  }
  const int q_len = a.cu_q[seq + 1] - a.cu_q[seq];
  if (i < 0 || i >= q_len || (a.expand_e > 0 && q_len > a.expand_e)) return -1;
  *table_row = seq;
  *query_row = a.cu_q[seq] + i;
  return clamp_length(a.lengths[seq] - q_len + i + 1, a);
}

// Maximum of an int over the wave: DPP within rows of 16 lanes, then the 4
// row results through scalar reads (no LDS traffic).
__device__ __forceinline__ int wave_max_i(int x) {
  x = max(x, __builtin_amdgcn_update_dpp(0, x, kDppQuadXor1, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, kDppQuadXor2, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, kDppRowHalfMirror, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, kDppRowMirror, 0xF, 0xF, false));
  return max(max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
             max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

// The work of one row and HPW consecutive q heads of one kv head (the
// grouped-query heads that share it) over splits split0, split0 + step, ...
// of the row's partition: each K/V vector a lane loads serves all HPW heads.
// Multi-split rows write (m, l, acc) partials, single splits the output; a
// zero-length row writes zeros (from split 0).
template <typename T, int VEC, int LPT, int HPW>
__device__ __forceinline__ void decode_work(const DecodeArgs& a, int64_t row, int head0,
                                            int split0, int step) {
  // Loads per chunk: fewer when many heads' state shares the registers.
  constexpr int U = (2 * kU / HPW) < 1 ? 1 : ((2 * kU / HPW) > kU ? kU : 2 * kU / HPW);
  constexpr int TPL = 64 / LPT;  // tokens per wave load
  constexpr int CH = U * TPL;    // tokens per chunk
  using raw_t = typename Vec<T, VEC>::raw_t;

  const int lane = threadIdx.x & 63;
  const int dg = lane % LPT;
  const int tg = lane / LPT;
  const int kvh = head0 / a.group;
  int64_t trow, qrow;
  const int n = row_length(row, a, &trow, &qrow);
  if (n < 0) return;
  const bool dvalid = dg * VEC < a.head_dim;
  T* out = reinterpret_cast<T*>(a.out) + qrow * a.o_row + (int64_t)head0 * a.o_head + dg * VEC;

  if (n == 0) {
    if (split0 == 0 && tg == 0 && dvalid) {
      float z[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) z[i] = 0.f;
#pragma unroll
      for (int h = 0; h < HPW; ++h) store_raw<T, VEC>(out + h * a.o_head, pack<T, VEC>(z));
    }
    return;
  }
  const Partition P = partition(n, a);
  if (split0 >= P.nsplit) return;
  // bf16 with 8-element vectors: the q.k product runs on packed bf16 pairs
  // (v_dot2 with fp32 accumulation, products exact in fp32) against the
  // unscaled q; the scale is applied to the reduced score.
  constexpr bool kDot2 = std::is_same<T, bf16_t>::value && VEC == 8;
  uint32_t qp2[HPW][VEC / 2];
  float qf[HPW][VEC];
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    if constexpr (kDot2) {
      const T* qp = reinterpret_cast<const T*>(a.q) + qrow * a.q_row +
                    (int64_t)(head0 + h) * a.q_head + dg * VEC;
      const raw_t r = dvalid ? load_raw<T, VEC>(qp) : raw_t{0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < VEC / 2; ++i) qp2[h][i] = r[i];
      continue;
    }
    const T* qp = reinterpret_cast<const T*>(a.q) + qrow * a.q_row +
                  (int64_t)(head0 + h) * a.q_head + dg * VEC;
    if (dvalid) {
      unpack<T, VEC>(load_raw<T, VEC>(qp), qf[h]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) qf[h][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) qf[h][i] *= a.scale_log2;
  }
  // Lanes past head_dim read dims [0, VEC) instead (in bounds); their q is zero
  // and they store nothing.
  const int lane_dim = dvalid ? dg * VEC : 0;
  const T* kbase = reinterpret_cast<const T*>(a.k) + (int64_t)kvh * a.k_head + lane_dim;
  const T* vbase = reinterpret_cast<const T*>(a.v) + (int64_t)kvh * a.v_head + lane_dim;
  const int32_t* table = a.tables + trow * a.table_stride;
  // Shared prefixes start at page 0: only rows whose first page is their
  // neighbour's compare further pages (two uniform loads otherwise).
  bool share_prev = false, share_next = false;
  {
    const int64_t table_rows = a.cu_q != nullptr ? (int64_t)a.num_seqs : a.rows;
    const int first = table[0];
    if (trow > 0) share_prev = table[-a.table_stride] == first;
    if (trow + 1 < table_rows) share_next = table[a.table_stride] == first;
  }

  // The split loop is instantiated twice: with the per-page sharing test and,
  // for rows that share no first page with a neighbour (all of a batch of
  // independent prompts), without it, so that such rows run no extra
  // instructions per chunk.
  auto run = [&](auto hint_c) {
    constexpr bool kHint = decltype(hint_c)::value;
    for (int split = split0; split < P.nsplit; split += step) {
      const int b0 = P.first + split * P.bps;
      const int b1 = min(b0 + P.bps, P.first + P.pages);
      const int tb = max(P.start, b0 * a.block_size);
      const int te = min(n, b1 * a.block_size);

      float m[HPW], l[HPW];
      float acc[HPW][VEC];
#pragma unroll
      for (int h = 0; h < HPW; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.f;
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[h][i] = 0.f;
      }

      for (int seg = b0; seg < b1; seg += 64) {
        const bool in_seg = seg + lane < b1;
        const int tbl = in_seg ? table[seg + lane] : 0;
        const int s_tb = max(tb, seg * a.block_size);
        const int s_te = min(te, (seg + 64) * a.block_size);
        if (s_tb >= s_te) continue;
        // Pages this row shares with a neighbouring row of the batch (the same
        // block at the same table index: parallel samples of one prompt, batches
        // grouped by prefix) are read with ordinary loads, so that the rows'
        // waves, dispatched together, find them in L2; other pages stream with
        // non-temporal loads. Only the cache policy depends on this.
        uint64_t shared_pages = 0;
        if constexpr (kHint) {
          bool shared = false;
          if (in_seg && share_prev) shared = table[seg + lane - a.table_stride] == tbl;
          if (in_seg && share_next) shared |= table[seg + lane + a.table_stride] == tbl;
          shared_pages = a.line_shared ? ~0ull : __ballot(shared);
        }
        // Branch-free loads: positions past the end re-read the last valid token
        // (masked out of the softmax), so a chunk is one straight run of loads.
        auto issue = [&](int p0, raw_t (&kr)[U], raw_t (&vr)[U], auto stream_c) {
          constexpr bool kStream = decltype(stream_c)::value;
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int pos = min(p0 + u * TPL + tg, s_te - 1);
            int page, off;
            if (a.bs_shift >= 0) {
              page = pos >> a.bs_shift;
              off = pos & (a.block_size - 1);
            } else {
              page = pos / a.block_size;
              off = pos - page * a.block_size;
            }
            const int64_t blk = shfl_i32(tbl, page - seg);
            if constexpr (kStream) {
              kr[u] = load_kv<T, VEC>(kbase + blk * a.k_block + (int64_t)off * a.k_token);
              vr[u] = load_kv<T, VEC>(vbase + blk * a.v_block + (int64_t)off * a.v_token);
            } else {
              kr[u] = load_raw<T, VEC>(kbase + blk * a.k_block + (int64_t)off * a.k_token);
              vr[u] = load_raw<T, VEC>(vbase + blk * a.v_block + (int64_t)off * a.v_token);
            }
          }
        };
        // The chunk at p0 is read with ordinary loads when one of its pages is
        // shared with a neighbouring row (wave-uniform).
        auto load_chunk = [&](int p0, raw_t (&kr)[U], raw_t (&vr)[U]) {
          if constexpr (kHint) {
            const int last = min(p0 + CH, s_te) - 1;
            int lo, hi;
            if (a.bs_shift >= 0) {
              lo = (p0 >> a.bs_shift) - seg;
              hi = (last >> a.bs_shift) - seg;
            } else {
              lo = p0 / a.block_size - seg;
              hi = last / a.block_size - seg;
            }
            const uint64_t span = hi - lo >= 63 ? ~0ull : ((2ull << (hi - lo)) - 1);
            if ((shared_pages >> lo) & span) {
              issue(p0, kr, vr, std::false_type{});
              return;
            }
          }
          issue(p0, kr, vr, std::true_type{});
        };
        raw_t kr[U], vr[U];
        load_chunk(s_tb, kr, vr);
        for (int p0 = s_tb; p0 < s_te; p0 += CH) {
          float sc[HPW][U];
          float mx[HPW];
#pragma unroll
          for (int h = 0; h < HPW; ++h) mx[h] = m[h];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            float kf[VEC];
            if constexpr (!kDot2) unpack<T, VEC>(kr[u], kf);
            const bool visible = p0 + u * TPL + tg < s_te;
#pragma unroll
            for (int h = 0; h < HPW; ++h) {
              float d = 0.f;
              if constexpr (kDot2) {
#pragma unroll
                for (int i = 0; i < VEC / 2; ++i)
                  d = __builtin_amdgcn_fdot2_f32_bf16(
                      __builtin_bit_cast(bf16x2_t, qp2[h][i]),
                      __builtin_bit_cast(bf16x2_t, (uint32_t)kr[u][i]), d, false);
                d = group_sum<LPT>(d) * a.scale_log2;
              } else {
#pragma unroll
                for (int i = 0; i < VEC; ++i) d = fmaf(qf[h][i], kf[i], d);
                d = group_sum<LPT>(d);
              }
              sc[h][u] = visible ? d : -INFINITY;
              mx[h] = fmaxf(mx[h], sc[h][u]);
            }
          }
          float safe[HPW];
#pragma unroll
          for (int h = 0; h < HPW; ++h) {
            safe[h] = (mx[h] == -INFINITY) ? 0.f : mx[h];
            const float corr = fast_exp2(m[h] - safe[h]);
            l[h] *= corr;
#pragma unroll
            for (int i = 0; i < VEC; ++i) acc[h][i] *= corr;
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
            float vf[VEC];
            unpack<T, VEC>(vr[u], vf);
#pragma unroll
            for (int h = 0; h < HPW; ++h) {
              const float p = fast_exp2(sc[h][u] - safe[h]);
              l[h] += p;
#pragma unroll
              for (int i = 0; i < VEC; ++i) acc[h][i] = fmaf(p, vf[i], acc[h][i]);
            }
          }
#pragma unroll
          for (int h = 0; h < HPW; ++h) m[h] = mx[h];
          if (p0 + CH < s_te) load_chunk(p0 + CH, kr, vr);
        }
      }

#pragma unroll
      for (int h = 0; h < HPW; ++h) {
        // Merge the token groups' states (fixed butterfly order).
        const float M = cross_group_max<LPT>(m[h]);
        const float w = (m[h] == -INFINITY) ? 0.f : fast_exp2(m[h] - M);
        const float L = cross_group_sum<LPT>(l[h] * w);
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[h][i] = cross_group_sum<LPT>(acc[h][i] * w);

        if (P.nsplit == 1) {
          if (tg == 0 && dvalid) {
            const float inv = fast_rcp(fmaxf(L, 1e-30f));
            float o[VEC];
#pragma unroll
            for (int i = 0; i < VEC; ++i) o[i] = acc[h][i] * inv;
            store_raw<T, VEC>(out + h * a.o_head, pack<T, VEC>(o));
          }
        } else {
          const int64_t idx = ((row * a.q_heads + head0 + h) * kMaxSplits) + split;
          if (lane == 0) {
            a.part_ml[idx * 2 + 0] = M;
            a.part_ml[idx * 2 + 1] = L;
          }
          if (tg == 0 && dvalid) {
            float* dst = a.part_acc + idx * a.head_dim + dg * VEC;
#pragma unroll
            for (int i = 0; i < VEC; ++i) dst[i] = acc[h][i];
          }
        }
      }
    }
  };
  if (share_prev || share_next || a.line_shared) {
    run(std::true_type{});
    return;
  }
  run(std::false_type{});
}

// Grid slot of this wave: its row (after the longest-first ranking) and its
// first split (rotated). False when the slot has no row.
__device__ __forceinline__ bool grid_slot(const DecodeArgs& a, int64_t& row, int& split0) {
  row = a.row_base + blockIdx.z;
  // Longest splits first: within each group of 64 consecutive rows, grid
  // row slot z takes the row of rank z by split length (pages per split,
  // descending; ties keep row order, so rows whose splits are equally long,
  // e.g. neighbours sharing a prefix, stay together). Workgroups are
  // dispatched in slot order, so the long splits start first and the drain
  // at the end of the launch is made of short ones. Every wave of the group
  // ranks the same 64 rows (one coalesced load; the compare loop only runs
  // when the split lengths differ), so no extra launch is needed.
  if (a.cu_q == nullptr) {
    const int lane = threadIdx.x & 63;
    const int64_t g0 = row - (blockIdx.z & 63);
    const int64_t mine = g0 + lane;
    int key = -1;
    if (mine < a.rows) {
      const int n = clamp_length(a.lengths[mine], a);
      key = n > 0 ? partition(n, a).bps : 0;
    }
    const int slot = (int)(blockIdx.z & 63);
    // Rank only when the group's split lengths differ by 2x or more: only then
    // does the order shorten the drain (and rows of equal split length, such
    // as rows sharing a prefix, keep their dispatch neighbourhood). kmin is
    // the smallest key of the group's rows (lanes past the last row are left
    // out); a zero-length row makes it 0, so such a group is always ranked.
    const int kmax = wave_max_i(key);
    const int kmin = -wave_max_i(key >= 0 ? -key : INT32_MIN + 1);
    if (kmax >= 2 * kmin) {
      int rank = 0;
#pragma unroll
      for (int j = 0; j < 64; ++j) {
        const int other = __builtin_amdgcn_readlane(key, j);
        rank += (other > key) || (other == key && j < lane);
      }
      const uint64_t hit = __ballot(rank == slot && key >= 0);
      if (hit == 0) return false;  // slot past the last row of a partial group
      row = g0 + __builtin_ffsll((long long)hit) - 1;
    }
  }
  // Workgroup L = x + gx * (head + heads * row) runs on XCD L % 8. Rows need
  // different split counts, so with split = x the low split indices (present
  // in every row) would pile onto the same XCDs; rotating the split index by
  // (head + heads * row) spreads every split position evenly over the XCDs.
  split0 = (int)blockIdx.x - (int)((blockIdx.y + (int64_t)gridDim.y * blockIdx.z) % gridDim.x);
  if (split0 < 0) split0 += gridDim.x;
  return true;
}

// Grid form: one wave per (split column, group of HPW q heads, row).
template <typename T, int VEC, int LPT, int HPW>
__global__ __launch_bounds__(64) void paged_decode_kernel(DecodeArgs a) {
  int64_t row;
  int split0;
  if (!grid_slot(a, row, split0)) return;
  decode_work<T, VEC, LPT, HPW>(a, row, (int)blockIdx.y * HPW, split0, gridDim.x);
}

// ------------------------------------------------ grouped-query heads on MFMA
// One wave per (split column, kv head, row) serves all `group` (3..16) q heads
// of the kv head with v_mfma_f32_16x16x32 tiles:
//  * S = K Q^T per 16 tokens: A = K (lane l: token l % 16, dims 32c + 8(l / 16)
//    .. +7, one 16-byte load straight from the page), B = Q^T of the group
//    (lane l: q head l % 16, same dims; columns past the group are zero).
//    The accumulator lane l holds head l % 16 at tokens 4(l / 16) .. +3.
//  * Online softmax per head column in the log2 domain (max over the 4 lane
//    groups of a column with two shuffles; reference max moved only when a
//    score exceeds it by more than 8, as in the prefill kernel).
//  * O^T = V^T P^T per 32 tokens: the two S accumulators of a lane, rounded to
//    the storage dtype, are its P^T B-operand (tokens 4g .. +3 and 16 + 4g ..
//    +3 of the chunk); V goes through a wave-private LDS tile (row-major,
//    XOR-swizzled 16-byte chunks) and ds_read_b64_tr_b16 returns the V^T
//    A-operand with the same token slots.
//  * Partition, split rotation, longest-first order and partials are those of
//    the VALU kernel, so the same merge kernel combines the splits.
constexpr int kMfmaAllGroups = 8;  // groups this large always take the MFMA kernel
constexpr int kMfmaMinGroup = 3;    // smaller groups use the VALU kernel
constexpr int kMfmaHeads = 16;      // q heads per tile (MFMA columns)
constexpr int kMfmaChunk = 32;      // tokens per PV step

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

template <typename T>
struct Mfma16;
template <>
struct Mfma16<bf16_t> {
  __device__ static f32x4_t run(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma16<f16_t> {
  __device__ static f32x4_t run(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
};

// Element offset of dim d of token row r in the LDS V tile: the 16-byte chunk
// index is XOR-swizzled by the row (D = 128: 16 chunks per row; D = 64: 8).
template <int D>
__device__ __forceinline__ int vt_at(int r, int d) {
  constexpr int KCH = D / 8;
  int swz;
  if constexpr (KCH == 16) swz = ((r & 3) << 2) ^ ((r >> 2) & 3);
  else swz = (((r >> 1) & 1) << 2) ^ ((r >> 2) & 3);
  return r * D + (((d >> 3) ^ swz) << 3) + (d & 7);
}

// ds_read_b64_tr_b16: within each 16-lane group, lane j receives element j % 4
// of the 8-byte chunks addressed by lanes 4i + j / 4 (element i of the result).
__device__ __forceinline__ u32x2_t lds_tr16(const uint16_t* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (v4s __attribute__((address_space(3)))*)(const_cast<uint16_t*>(p)));
  return __builtin_bit_cast(u32x2_t, r);
}

template <typename T, int D>
__device__ __forceinline__ void decode_work_mfma(const DecodeArgs& a, int64_t row, int head0,
                                                 int split0, int step, uint16_t* vt) {
  constexpr int DC = D / 32;           // 32-dim k chunks of S = K Q^T
  constexpr int DT = D / 16;           // 16-dim tiles of O^T
  constexpr int KCH = D / 8;           // 16-byte chunks per token row
  constexpr int RPI = 64 / KCH;        // token rows per V staging instruction
  constexpr int NV = kMfmaChunk / RPI; // V staging loads per chunk
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int kvh = head0 / a.group;
  int64_t trow, qrow;
  const int n = row_length(row, a, &trow, &qrow);
  if (n < 0) return;
  const bool hcol = col < a.group;
  T* out = reinterpret_cast<T*>(a.out) + qrow * a.o_row + (int64_t)(head0 + col) * a.o_head +
           4 * grp;
  if (n == 0) {
    if (split0 == 0 && hcol) {
#pragma unroll
      for (int t = 0; t < DT; ++t) *reinterpret_cast<u32x2_t*>(out + 16 * t) = u32x2_t{0u, 0u};
    }
    return;
  }
  const Partition P = partition(n, a);
  if (split0 >= P.nsplit) return;

  u32x4_t qop[DC];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + qrow * a.q_row +
                  (int64_t)(head0 + (hcol ? col : 0)) * a.q_head + 8 * grp;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(qp + 32 * c);
      qop[c] = hcol ? v : u32x4_t{0u, 0u, 0u, 0u};
    }
  }
  const T* kbase = reinterpret_cast<const T*>(a.k) + (int64_t)kvh * a.k_head + 8 * grp;
  // V staging: instruction r loads token rows RPI r .. + RPI - 1 straight
  // into LDS (lane l's 16 bytes land at row RPI r + l / KCH, slot l % KCH), so
  // the lane fetches the chunk stored at that slot: slot ^ swizzle(row). The
  // swizzle depends on row % 16 and RPI * r repeats it every 16 / RPI
  // instructions.
  const int v_row = lane / KCH;
  constexpr int SWP = 16 / RPI < NV ? 16 / RPI : NV;  // distinct swizzles
  const T* vbase[SWP];
#pragma unroll
  for (int r = 0; r < SWP; ++r) {
    const int row = v_row + RPI * r;
    vbase[r] = reinterpret_cast<const T*>(a.v) + (int64_t)kvh * a.v_head +
               (vt_at<D>(row, 8 * (lane % KCH)) - row * D);
  }
  // The chunk index the swizzle yields is the element offset's chunk part:
  // vt_at(row, 8 s) - row D is 8 (s ^ swizzle(row)), an involution, so the
  // lane's global chunk is the one vt_at maps its slot to.
  const uint32_t vt_lds = lds_offset(vt);
  const int32_t* table = a.tables + trow * a.table_stride;
  // Transposed reads of tile t, token half h: rows 16h + 4grp + (col >> 2),
  // dims 16t + 4(col & 3); half 1 is 16 rows (16 D elements) further.
  uint32_t tr_off[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) tr_off[t] = vt_at<D>(4 * grp + (col >> 2), 16 * t + 4 * (col & 3));

  auto page_addr = [&](int pos, int tbl, int seg, int64_t blk_stride, int64_t tok_stride) {
    int page, off;
    if (a.bs_shift >= 0) {
      page = pos >> a.bs_shift;
      off = pos & (a.block_size - 1);
    } else {
      page = pos / a.block_size;
      off = pos - page * a.block_size;
    }
    const int64_t blk = shfl_i32(tbl, page - seg);
    return blk * blk_stride + (int64_t)off * tok_stride;
  };

  for (int split = split0; split < P.nsplit; split += step) {
    const int b0 = P.first + split * P.bps;
    const int b1 = min(b0 + P.bps, P.first + P.pages);
    const int tb = max(P.start, b0 * a.block_size);
    const int te = min(n, b1 * a.block_size);
    float m = -1e30f;  // reference max (log2 domain) of this lane's head column
    float lsum = 0.f;  // partial sum over this lane's token slots
    f32x4_t acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int seg = b0; seg < b1; seg += 64) {
      const int tbl = (seg + lane < b1) ? table[seg + lane] : 0;
      const int s_tb = max(tb, seg * a.block_size);
      const int s_te = min(te, (seg + 64) * a.block_size);
      for (int p0 = s_tb; p0 < s_te; p0 += kMfmaChunk) {
        // Loads (branch-free: positions past the end re-read the last token).
        // The A-operand layout gives each token 4 lanes (64 bytes) per
        // instruction, so instructions c and c + 1 read the two halves of one
        // 128-byte line: ordinary (L1-allocating) loads let the second half
        // hit the line the first brought in.
        u32x4_t kop[2][DC];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int pos = min(p0 + 16 * t + col, s_te - 1);
          const T* kp = kbase + page_addr(pos, tbl, seg, a.k_block, a.k_token);
#pragma unroll
          for (int c = 0; c < DC; ++c) kop[t][c] = *reinterpret_cast<const u32x4_t*>(kp + 32 * c);
        }
        // V straight into the LDS tile. The previous chunk's transposed reads
        // have returned (its PV MFMAs consumed them), so the tile is free.
#pragma unroll
        for (int r = 0; r < NV; ++r) {
          const int pos = min(p0 + v_row + RPI * r, s_te - 1);
          const T* vp = vbase[r % SWP] + page_addr(pos, tbl, seg, a.v_block, a.v_token);
          lds_dma16(vp, __builtin_amdgcn_readfirstlane(vt_lds + 1024 * r));
        }
        // S tiles and their masked max (tokens p0 + 16t + 4grp + i).
        f32x4_t sc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          sc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int c = 0; c < DC; ++c) sc[t] = Mfma16<T>::run(kop[t][c], qop[c], sc[t]);
        }
        const int lim = s_te - p0 - 4 * grp;  // token slot t*16 + i visible when < lim
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x = 16 * t + i < lim ? sc[t][i] * a.scale_log2 : -INFINITY;
            sc[t][i] = x;
            mx = fmaxf(mx, x);
          }
        mx = fmaxf(mx, shfl_xor_f32(mx, 16));
        mx = fmaxf(mx, shfl_xor_f32(mx, 32));
        if (__any(mx > m + 8.f)) {
          const float mnew = fmaxf(m, mx);
          const float corr = fast_exp2(m - mnew);
          lsum *= corr;
#pragma unroll
          for (int t = 0; t < DT; ++t) acc[t] *= corr;
          m = mnew;
        }
        float p[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            p[t][i] = fast_exp2(sc[t][i] - m);
            lsum += p[t][i];
          }
        const u32x4_t pop = u32x4_t{pack2<T>(p[0][0], p[0][1]), pack2<T>(p[0][2], p[0][3]),
                                    pack2<T>(p[1][0], p[1][1]), pack2<T>(p[1][2], p[1][3])};
        vm_wait<0>();  // the V tile has landed
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const u32x2_t lo = lds_tr16(vt + tr_off[t]);
          const u32x2_t hi = lds_tr16(vt + tr_off[t] + 16 * D);
          acc[t] = Mfma16<T>::run(u32x4_t{lo[0], lo[1], hi[0], hi[1]}, pop, acc[t]);
        }
      }
    }
    const float L = lsum + shfl_xor_f32(lsum, 16);
    const float L4 = L + shfl_xor_f32(L, 32);
    if (P.nsplit == 1) {
      if (hcol) {
        const float inv = fast_rcp(fmaxf(L4, 1e-30f));
#pragma unroll
        for (int t = 0; t < DT; ++t)
          *reinterpret_cast<u32x2_t*>(out + 16 * t) =
              u32x2_t{pack2<T>(acc[t][0] * inv, acc[t][1] * inv),
                      pack2<T>(acc[t][2] * inv, acc[t][3] * inv)};
      }
    } else if (hcol) {
      const int64_t idx = ((row * a.q_heads + head0 + col) * kMaxSplits) + split;
      if (grp == 0) {
        a.part_ml[idx * 2 + 0] = m;
        a.part_ml[idx * 2 + 1] = L4;
      }
      float* dst = a.part_acc + idx * a.head_dim + 4 * grp;
#pragma unroll
      for (int t = 0; t < DT; ++t) *reinterpret_cast<f32x4_t*>(dst + 16 * t) = acc[t];
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(64) void paged_decode_mfma_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t vt[kMfmaChunk * D];
  int64_t row;
  int split0;
  if (!grid_slot(a, row, split0)) return;
  decode_work_mfma<T, D>(a, row, (int)blockIdx.y * a.group, split0, gridDim.x, vt);
}

// Log-sum-exp merge of one (row, q head)'s split partials by one wave, for
// head dims [d0, d0 + 64 * ND): lane s holds split s's weight; each lane owns
// ND dims and issues the loads of all splits at once, then combines them in
// split order.
template <typename T, int ND>
__device__ __forceinline__ void merge_partials(const DecodeArgs& a, int64_t row, int head,
                                               int64_t qrow, int nsplit, int lane, int d0) {
  const int64_t idx0 = (row * a.q_heads + head) * kMaxSplits;
  const bool live = lane < nsplit;
  const float mi = live ? a.part_ml[(idx0 + lane) * 2 + 0] : -INFINITY;
  const float li = live ? a.part_ml[(idx0 + lane) * 2 + 1] : 0.f;
  const float M = wave_max(mi);
  const float wi = live ? fast_exp2(mi - M) : 0.f;
  const float L = wave_sum(wi * li);
  const float inv = fast_rcp(fmaxf(L, 1e-30f));
  const float* part = a.part_acc + idx0 * a.head_dim;
  float acc[ND];
#pragma unroll
  for (int e = 0; e < ND; ++e) acc[e] = 0.f;
  float v[kMaxSplits][ND];
#pragma unroll
  for (int j = 0; j < kMaxSplits; ++j)
#pragma unroll
    for (int e = 0; e < ND; ++e) {
      const int d = d0 + lane + 64 * e;
      v[j][e] = (j < nsplit && d < a.head_dim) ? part[(int64_t)j * a.head_dim + d] : 0.f;
    }
#pragma unroll
  for (int j = 0; j < kMaxSplits; ++j) {
    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wi), j));
#pragma unroll
    for (int e = 0; e < ND; ++e) acc[e] = fmaf(w, v[j][e], acc[e]);
  }
  T* out = reinterpret_cast<T*>(a.out) + qrow * a.o_row + (int64_t)head * a.o_head;
#pragma unroll
  for (int e = 0; e < ND; ++e) {
    const int d = d0 + lane + 64 * e;
    if (d < a.head_dim) out[d] = from_f32<T>(acc[e] * inv);
  }
}

// Log-sum-exp merge of a row's split partials, one wave per (row, q head),
// 4 waves per workgroup.
template <typename T, int ND>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const int head = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (head >= a.q_heads) return;
  const int64_t row = a.row_base + blockIdx.y;
  int64_t trow, qrow;
  const int n = row_length(row, a, &trow, &qrow);
  if (n <= 0) return;
  const Partition P = partition(n, a);
  if (P.nsplit <= 1) return;
  merge_partials<T, ND>(a, row, head, qrow, P.nsplit, lane, 0);
}

template <typename T>
void launch_merge(int head_dim, dim3 grid, hipStream_t s, const DecodeArgs& a) {
  if (head_dim <= 64) {
    hipLaunchKernelGGL((paged_decode_merge_kernel<T, 1>), grid, dim3(256), 0, s, a);
  } else if (head_dim <= 128) {
    hipLaunchKernelGGL((paged_decode_merge_kernel<T, 2>), grid, dim3(256), 0, s, a);
  } else if (head_dim <= 256) {
    hipLaunchKernelGGL((paged_decode_merge_kernel<T, 4>), grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((paged_decode_merge_kernel<T, 8>), grid, dim3(256), 0, s, a);
  }
}

template <typename T, int VEC, int LPT>
bool launch_hpw(int hpw, dim3 grid, hipStream_t s, const DecodeArgs& a) {
  switch (hpw) {
    case 1: hipLaunchKernelGGL((paged_decode_kernel<T, VEC, LPT, 1>), grid, dim3(64), 0, s, a); return true;
    case 2: hipLaunchKernelGGL((paged_decode_kernel<T, VEC, LPT, 2>), grid, dim3(64), 0, s, a); return true;
    case 4: hipLaunchKernelGGL((paged_decode_kernel<T, VEC, LPT, 4>), grid, dim3(64), 0, s, a); return true;
    case 8: hipLaunchKernelGGL((paged_decode_kernel<T, VEC, LPT, 8>), grid, dim3(64), 0, s, a); return true;
    default: return false;
  }
}

// Instantiations: every (VEC, LPT) for one head per wave; grouped heads per
// wave (HPW > 1) only for full-width lanes of the usual head dims
// (16-byte vectors, LPT 4, 8 or 16: head_dim 32, 64, 128 in 16-bit types).
template <typename T, int VEC>
bool launch_vec(int lpt, int hpw, dim3 grid, hipStream_t s, const DecodeArgs& a) {
  constexpr bool kWide = VEC * (int)sizeof(T) == 16;
  switch (lpt) {
#define VRH_LPT(L)                                                                 \
  case L:                                                                          \
    if (hpw == 1) {                                                                \
      hipLaunchKernelGGL((paged_decode_kernel<T, VEC, L, 1>), grid, dim3(64), 0, s, a); \
      return true;                                                                 \
    }                                                                              \
    if constexpr (kWide && L >= 4 && L <= 16) return launch_hpw<T, VEC, L>(hpw, grid, s, a); \
    return false;
    VRH_LPT(1)
    VRH_LPT(2)
    VRH_LPT(4)
    VRH_LPT(8)
    VRH_LPT(16)
    VRH_LPT(32)
    VRH_LPT(64)
#undef VRH_LPT
    default: return false;
  }
}

template <typename T>
bool launch_decode(int vec, int lpt, int hpw, dim3 grid, hipStream_t s, const DecodeArgs& a) {
  switch (vec) {
    case 1: return launch_vec<T, 1>(lpt, hpw, grid, s, a);
    case 2: return launch_vec<T, 2>(lpt, hpw, grid, s, a);
    case 4: return launch_vec<T, 4>(lpt, hpw, grid, s, a);
    case 8:
      if constexpr (sizeof(T) == 2) return launch_vec<T, 8>(lpt, hpw, grid, s, a);
      return false;
    default: return false;
  }
}

}  // namespace
}  // namespace vrh

using namespace vrh;


extern "C" size_t vrh_paged_decode_workspace_bytes(int64_t rows, int32_t q_heads,
                                                   int32_t head_dim) {
  if (rows <= 0 || q_heads <= 0 || head_dim <= 0) return 0;
  const size_t parts = (size_t)rows * q_heads * kMaxSplits;
  const size_t ml = (parts * 2 * sizeof(float) + 255) & ~(size_t)255;
  return ml + parts * head_dim * sizeof(float);
}

// Shared launcher of the decode kernels. `workspace` == nullptr forces one
// split per row (used by the packed-prefill expansion, which has no workspace).
int vrh_decode_rows(int dtype, void* out, const void* q, const void* key_cache,
                    const void* value_cache, const int32_t* block_tables,
                    const int32_t* context_lengths, const int32_t* cu_q, int32_t num_seqs,
                    int32_t expand_e, int64_t rows, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                    int32_t block_size, int32_t table_width, int64_t table_stride,
                    int64_t q_row_stride, int64_t q_head_stride, int64_t out_row_stride,
                    int64_t out_head_stride, int64_t k_block_stride, int64_t k_token_stride,
                    int64_t k_head_stride, int64_t v_block_stride, int64_t v_token_stride,
                    int64_t v_head_stride, int32_t window, void* workspace,
                    size_t workspace_bytes, hipStream_t s, const char* who) {
  const int es = dtype_bytes(dtype);
  VRH_CHECK_ARG(es > 0, "%s: unknown dtype %d", who, dtype);
  VRH_CHECK_ARG(rows >= 0 && q_heads >= 1 && kv_heads >= 1 && q_heads % kv_heads == 0,
                "%s: query heads must be a positive multiple of KV heads", who);
  VRH_CHECK_ARG(head_dim >= 1 && head_dim <= 512, "%s: head_dim %d unsupported", who,
                head_dim);
  VRH_CHECK_ARG(block_size >= 1 && table_width >= 0 && window >= 0,
                "%s: bad block_size/table_width/window", who);
  VRH_CHECK_ARG(q_heads <= 65535, "%s: too many heads", who);
  if (rows == 0) return VRH_OK;
  VRH_CHECK_ARG(out && q && key_cache && value_cache && context_lengths &&
                    (block_tables || table_width == 0),
                "%s: null pointer", who);
  if (workspace != nullptr) {
    const size_t need = vrh_paged_decode_workspace_bytes(rows, q_heads, head_dim);
    VRH_CHECK_ARG(workspace_bytes >= need, "%s: workspace of %zu bytes needed, %zu given", who,
                  need, workspace_bytes);
    VRH_CHECK_ARG(((uintptr_t)workspace & 255) == 0, "%s: workspace misaligned", who);
  }

  // Widest per-lane vector (<= 16 B) that divides head_dim and keeps every
  // access aligned.
  int vec = 16 / es;
  auto aligned = [&](int v) {
    const int64_t vs[] = {q_row_stride, q_head_stride, out_row_stride, out_head_stride,
                          k_block_stride, k_token_stride, k_head_stride, v_block_stride,
                          v_token_stride, v_head_stride};
    if (head_dim % v) return false;
    for (int64_t st : vs)
      if (st % v) return false;
    const void* ps[] = {out, q, key_cache, value_cache};
    for (const void* p : ps)
      if ((uintptr_t)p % ((size_t)v * es)) return false;
    return true;
  };
  while (vec > 1 && !aligned(vec)) vec >>= 1;
  int lpt = 1;
  while (lpt * vec < head_dim) lpt <<= 1;
  VRH_CHECK_ARG(lpt <= 64, "%s: head_dim %d too large for dtype", who, head_dim);

  DecodeArgs a;
  a.out = out;
  a.q = q;
  a.k = key_cache;
  a.v = value_cache;
  a.tables = block_tables;
  a.lengths = context_lengths;
  a.rows = rows;
  a.part_ml = nullptr;
  a.part_acc = nullptr;
  if (workspace != nullptr) {
    const size_t parts = (size_t)rows * q_heads * kMaxSplits;
    a.part_ml = (float*)workspace;
    a.part_acc = (float*)((char*)workspace + ((parts * 2 * sizeof(float) + 255) & ~(size_t)255));
  }
  a.q_row = q_row_stride;
  a.q_head = q_head_stride;
  a.o_row = out_row_stride;
  a.o_head = out_head_stride;
  a.k_block = k_block_stride;
  a.k_token = k_token_stride;
  a.k_head = k_head_stride;
  a.v_block = v_block_stride;
  a.v_token = v_token_stride;
  a.v_head = v_head_stride;
  a.table_stride = table_stride;
  a.cu_q = cu_q;
  a.num_seqs = num_seqs;
  a.expand_e = expand_e;
  a.q_heads = q_heads;
  a.group = q_heads / kv_heads;
  a.head_dim = head_dim;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.window = window;
  a.table_width = table_width;
  a.line_shared = ((int64_t)head_dim * es) % 128 != 0;
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)head_dim));
  // Pages per split: at least kSplitTokens tokens; without a workspace every
  // row is a single split (pages can never exceed the table width).
  a.min_bps = workspace != nullptr ? std::max(1, kSplitTokens / block_size)
                                   : std::max(1, table_width);

  // Grouped-query heads per wave: the largest of 8, 4, 2 dividing the group
  // (1 without grouping, or where no grouped instantiation exists).
  int hpw = 1;
  if (vec * es == 16 && lpt >= 4 && lpt <= 16)
    for (int h : {8, 4, 2})
      if (a.group % h == 0 && h <= kMaxHpw) {
        hpw = h;
        break;
      }
  // Grouped-query heads in 16-bit types with head_dim 64 or 128 (16-byte
  // aligned strides) run on the MFMA kernel when the group has 8 to 16 heads,
  // or 3 to 7 heads that the VALU kernel cannot serve from one wave (it would
  // re-read K/V); groups of 2 and 4 stay on the VALU kernel, which is as fast
  // there (measured: 4 heads per wave 454 against 496 us at 256 rows).
  const bool mfma_gqa = (dtype == VRH_DTYPE_BF16 || dtype == VRH_DTYPE_F16) && vec * es == 16 &&
                        (head_dim == 64 || head_dim == 128) && a.group >= kMfmaMinGroup &&
                        a.group <= kMfmaHeads && (a.group >= kMfmaAllGroups || hpw < a.group);
  // Largest split count any row of this table width can need: the grid is a
  // function of shapes only (graph capture), never of device lengths.
  const int max_pages = std::max(1, table_width);
  const int gx = std::max(1, std::min(kMaxSplits, ceil_div(max_pages, a.min_bps)));
  // Rows per launch: the grid's z limit rounded down to whole 64-row groups
  // (the longest-first ranking works on aligned groups of 64 rows).
  constexpr int64_t kRowsPerLaunch = 65535 / 64 * 64;
  for (int64_t first = 0; first < rows; first += kRowsPerLaunch) {
    a.row_base = first;
    const unsigned count = (unsigned)std::min<int64_t>(rows - first, kRowsPerLaunch);
    bool ok = false;
    if (mfma_gqa) {
      dim3 grid((unsigned)gx, (unsigned)kv_heads, count);
      ok = true;
      if (dtype == VRH_DTYPE_BF16) {
        if (head_dim == 128) hipLaunchKernelGGL((paged_decode_mfma_kernel<bf16_t, 128>), grid, dim3(64), 0, s, a);
        else hipLaunchKernelGGL((paged_decode_mfma_kernel<bf16_t, 64>), grid, dim3(64), 0, s, a);
      } else {
        if (head_dim == 128) hipLaunchKernelGGL((paged_decode_mfma_kernel<f16_t, 128>), grid, dim3(64), 0, s, a);
        else hipLaunchKernelGGL((paged_decode_mfma_kernel<f16_t, 64>), grid, dim3(64), 0, s, a);
      }
    } else {
      dim3 grid((unsigned)gx, (unsigned)(q_heads / hpw), count);
      switch (dtype) {
        case VRH_DTYPE_F32: ok = launch_decode<float>(vec, lpt, hpw, grid, s, a); break;
        case VRH_DTYPE_F16: ok = launch_decode<f16_t>(vec, lpt, hpw, grid, s, a); break;
        case VRH_DTYPE_BF16: ok = launch_decode<bf16_t>(vec, lpt, hpw, grid, s, a); break;
      }
    }
    VRH_CHECK_ARG(ok, "%s: no kernel for vec=%d lanes=%d heads/wave=%d", who, vec, lpt, hpw);
    if (gx == 1) continue;  // every row is a single split: output already written
    dim3 mgrid((unsigned)ceil_div(q_heads, 4), count);
    switch (dtype) {
      case VRH_DTYPE_F32: launch_merge<float>(head_dim, mgrid, s, a); break;
      case VRH_DTYPE_F16: launch_merge<f16_t>(head_dim, mgrid, s, a); break;
      case VRH_DTYPE_BF16: launch_merge<bf16_t>(head_dim, mgrid, s, a); break;
    }
  }
  VRH_RETURN_LAUNCH(who);
}

extern "C" int vrh_paged_decode(int dtype, void* out, const void* q, const void* key_cache,
                                const void* value_cache, const int32_t* block_tables,
                                const int32_t* context_lengths, int64_t rows, int32_t q_heads,
                                int32_t kv_heads, int32_t head_dim, int32_t block_size,
                                int32_t table_width, int64_t table_stride, int64_t q_row_stride,
                                int64_t q_head_stride, int64_t out_row_stride,
                                int64_t out_head_stride, int64_t k_block_stride,
                                int64_t k_token_stride, int64_t k_head_stride,
                                int64_t v_block_stride, int64_t v_token_stride,
                                int64_t v_head_stride, int32_t window, void* workspace,
                                size_t workspace_bytes, vrh_stream_t stream) {
  VRH_CHECK_ARG(rows == 0 || workspace != nullptr, "vrh_paged_decode: workspace is required");
  return vrh_decode_rows(dtype, out, q, key_cache, value_cache, block_tables, context_lengths,
                         nullptr, 0, 0, rows, q_heads, kv_heads, head_dim, block_size, table_width,
                         table_stride, q_row_stride, q_head_stride, out_row_stride,
                         out_head_stride, k_block_stride, k_token_stride, k_head_stride,
                         v_block_stride, v_token_stride, v_head_stride, window, workspace,
                         workspace_bytes, (hipStream_t)stream, "vrh_paged_decode");
}
