// Paged single-query (decode) attention, split-KV, for gfx950.
//
// Reference semantics: kernels/paged_attention.py:12-71 (torch_paged_attention
// and the windowed variant): per row, keys/values gathered through the row's
// own block table, GQA head h reads kv head h / G, scores scaled by 1/sqrt(D),
// fp32 softmax, output rounded to the storage dtype, zero rows for length 0.
//
// Design (bandwidth-bound; every K/V byte is read exactly once per q head):
//  * One 64-lane wavefront per (split, q head, row). A split is a run of whole
//    pages: bps = max(min_bps, ceil(pages / kMaxSplits)) pages, so the
//    partition depends only on the row's own length -> batch invariance.
//  * Lane layout: LPT lanes cover one token's head_dim with VEC elements each
//    (16-byte global loads for bf16 D=128: LPT=16), so one wave-wide load
//    instruction fetches TPL = 64 / LPT tokens; U = 4 loads of K and 4 of V are
//    in flight per lane per chunk.
//  * The row's page ids for up to 64 pages sit in one VGPR (one per lane) and
//    are fetched with ds_bpermute, so the page table is read once per split.
//  * Each token group keeps its own online-softmax state (m, l, acc) in the
//    log2 domain; groups are merged once per split with cross-lane shuffles,
//    so the inner loop has no cross-row reductions. QK^T partial sums reduce
//    within a 16-lane row with DPP.
//  * Splits of multi-split rows write (m, l, acc) partials to the workspace;
//    a merge kernel combines them in split order (log-sum-exp). Single-split
//    rows write the output directly.
#include <algorithm>

#include "common.h"

namespace vrh {
namespace {

constexpr int kMaxSplits = 32;
constexpr int kSplitTokens = 256;  // minimum tokens per split (whole pages)
constexpr int kU = 4;              // wave loads per chunk for each of K and V

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
  // Packed-prefill expansion (null for decode): row r is query i of sequence
  // s with cu_q[s] <= r < cu_q[s+1]; it reads table row s with causal length
  // lengths[s] - q_len(s) + i + 1.
  const int32_t* cu_q;
  int32_t num_seqs;
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

// Visible length and table row of a query row (decode: itself).
__device__ __forceinline__ int row_length(int64_t row, const DecodeArgs& a, int64_t* table_row) {
  if (a.cu_q == nullptr) {
    *table_row = row;
    return clamp_length(a.lengths[row], a);
  }
  int lo = 0, hi = a.num_seqs - 1;  // last s with cu_q[s] <= row
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.cu_q[mid] <= row) lo = mid; else hi = mid - 1;
  }
  *table_row = lo;
  const int q_len = a.cu_q[lo + 1] - a.cu_q[lo];
  const int i = (int)(row - a.cu_q[lo]);
  return clamp_length(a.lengths[lo] - q_len + i + 1, a);
}

template <typename T, int VEC, int LPT>
__global__ __launch_bounds__(64) void paged_decode_kernel(DecodeArgs a) {
  constexpr int TPL = 64 / LPT;  // tokens per wave load
  constexpr int CH = kU * TPL;   // tokens per chunk
  using raw_t = typename Vec<T, VEC>::raw_t;

  const int lane = threadIdx.x;
  const int dg = lane % LPT;
  const int tg = lane / LPT;
  const int head = blockIdx.y;
  const int64_t row = a.row_base + blockIdx.z;
  const int kvh = head / a.group;
  int64_t trow;
  const int n = row_length(row, a, &trow);
  const bool dvalid = dg * VEC < a.head_dim;
  T* out = reinterpret_cast<T*>(a.out) + row * a.o_row + head * a.o_head + dg * VEC;

  if (n == 0) {
    if (blockIdx.x == 0 && tg == 0 && dvalid) {
      float z[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) z[i] = 0.f;
      store_raw<T, VEC>(out, pack<T, VEC>(z));
    }
    return;
  }
  const Partition P = partition(n, a);
  if ((int)blockIdx.x >= P.nsplit) return;

  float qf[VEC];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + row * a.q_row + head * a.q_head + dg * VEC;
    if (dvalid) {
      unpack<T, VEC>(load_raw<T, VEC>(qp), qf);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) qf[i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) qf[i] *= a.scale_log2;
  }
  const T* kbase = reinterpret_cast<const T*>(a.k) + kvh * a.k_head + dg * VEC;
  const T* vbase = reinterpret_cast<const T*>(a.v) + kvh * a.v_head + dg * VEC;
  const int32_t* table = a.tables + trow * a.table_stride;

  for (int split = blockIdx.x; split < P.nsplit; split += gridDim.x) {
    const int b0 = P.first + split * P.bps;
    const int b1 = min(b0 + P.bps, P.first + P.pages);
    const int tb = max(P.start, b0 * a.block_size);
    const int te = min(n, b1 * a.block_size);

    float m = -INFINITY, l = 0.f;
    float acc[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] = 0.f;

    for (int seg = b0; seg < b1; seg += 64) {
      const int tbl = (seg + lane < b1) ? table[seg + lane] : 0;
      const int s_tb = max(tb, seg * a.block_size);
      const int s_te = min(te, (seg + 64) * a.block_size);
      for (int p0 = s_tb; p0 < s_te; p0 += CH) {
        raw_t kr[kU], vr[kU];
        bool val[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int pos = p0 + u * TPL + tg;
          val[u] = pos < s_te;
          int page, off;
          if (a.bs_shift >= 0) {
            page = pos >> a.bs_shift;
            off = pos & (a.block_size - 1);
          } else {
            page = pos / a.block_size;
            off = pos - page * a.block_size;
          }
          const int blk = shfl_i32(tbl, val[u] ? page - seg : 0);
          if (val[u] && dvalid) {
            const int64_t b = (int64_t)blk;
            kr[u] = load_raw_stream<T, VEC>(kbase + b * a.k_block + off * a.k_token);
            vr[u] = load_raw_stream<T, VEC>(vbase + b * a.v_block + off * a.v_token);
          } else {
            kr[u] = raw_t{};
            vr[u] = raw_t{};
          }
        }
        float s[kU];
        float mx = m;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          float kf[VEC];
          unpack<T, VEC>(kr[u], kf);
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < VEC; ++i) d = fmaf(qf[i], kf[i], d);
          d = group_sum<LPT>(d);
          s[u] = val[u] ? d : -INFINITY;
          mx = fmaxf(mx, s[u]);
        }
        const float safe = (mx == -INFINITY) ? 0.f : mx;
        const float corr = exp2f(m - safe);
        l *= corr;
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[i] *= corr;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const float p = exp2f(s[u] - safe);
          l += p;
          float vf[VEC];
          unpack<T, VEC>(vr[u], vf);
#pragma unroll
          for (int i = 0; i < VEC; ++i) acc[i] = fmaf(p, vf[i], acc[i]);
        }
        m = mx;
      }
    }

    // Merge the token groups' states (fixed butterfly order).
    const float M = cross_group_max<LPT>(m);
    const float w = (m == -INFINITY) ? 0.f : exp2f(m - M);
    const float L = cross_group_sum<LPT>(l * w);
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] = cross_group_sum<LPT>(acc[i] * w);

    if (P.nsplit == 1) {
      if (tg == 0 && dvalid) {
        const float inv = 1.f / fmaxf(L, 1e-30f);
        float o[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) o[i] = acc[i] * inv;
        store_raw<T, VEC>(out, pack<T, VEC>(o));
      }
    } else {
      const int64_t idx = ((row * a.q_heads + head) * kMaxSplits) + split;
      if (lane == 0) {
        a.part_ml[idx * 2 + 0] = M;
        a.part_ml[idx * 2 + 1] = L;
      }
      if (tg == 0 && dvalid) {
        float* dst = a.part_acc + idx * a.head_dim + dg * VEC;
#pragma unroll
        for (int i = 0; i < VEC; ++i) dst[i] = acc[i];
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(64) void paged_decode_merge_kernel(DecodeArgs a) {
  __shared__ float weights[kMaxSplits];
  const int lane = threadIdx.x;
  const int head = blockIdx.x;
  const int64_t row = a.row_base + blockIdx.y;
  int64_t trow;
  const int n = row_length(row, a, &trow);
  if (n == 0) return;
  const Partition P = partition(n, a);
  if (P.nsplit <= 1) return;
  const int64_t idx0 = (row * a.q_heads + head) * kMaxSplits;
  const bool live = lane < P.nsplit;
  const float mi = live ? a.part_ml[(idx0 + lane) * 2 + 0] : -INFINITY;
  const float li = live ? a.part_ml[(idx0 + lane) * 2 + 1] : 0.f;
  const float M = wave_max(mi);
  const float wi = live ? exp2f(mi - M) : 0.f;
  const float L = wave_sum(wi * li);
  if (lane < kMaxSplits) weights[lane] = wi;
  __syncthreads();
  const float inv = 1.f / fmaxf(L, 1e-30f);
  T* out = reinterpret_cast<T*>(a.out) + row * a.o_row + head * a.o_head;
  for (int d = lane; d < a.head_dim; d += 64) {
    float acc = 0.f;
    for (int s = 0; s < P.nsplit; ++s) acc = fmaf(weights[s], a.part_acc[(idx0 + s) * a.head_dim + d], acc);
    out[d] = from_f32<T>(acc * inv);
  }
}

template <typename T, int VEC>
bool launch_vec(int lpt, dim3 grid, hipStream_t s, const DecodeArgs& a) {
  switch (lpt) {
#define VRH_LPT(L)                                                                       \
  case L:                                                                                \
    hipLaunchKernelGGL((paged_decode_kernel<T, VEC, L>), grid, dim3(64), 0, s, a); \
    return true;
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
bool launch_decode(int vec, int lpt, dim3 grid, hipStream_t s, const DecodeArgs& a) {
  switch (vec) {
    case 1: return launch_vec<T, 1>(lpt, grid, s, a);
    case 2: return launch_vec<T, 2>(lpt, grid, s, a);
    case 4: return launch_vec<T, 4>(lpt, grid, s, a);
    case 8:
      if constexpr (sizeof(T) == 2) return launch_vec<T, 8>(lpt, grid, s, a);
      return false;
    default: return false;
  }
}

int dtype_size(int dtype) {
  return dtype == VRH_DTYPE_F32 ? 4 : (dtype == VRH_DTYPE_F16 || dtype == VRH_DTYPE_BF16) ? 2 : 0;
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
                    int64_t rows, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                    int32_t block_size, int32_t table_width, int64_t table_stride,
                    int64_t q_row_stride, int64_t q_head_stride, int64_t out_row_stride,
                    int64_t out_head_stride, int64_t k_block_stride, int64_t k_token_stride,
                    int64_t k_head_stride, int64_t v_block_stride, int64_t v_token_stride,
                    int64_t v_head_stride, int32_t window, void* workspace,
                    size_t workspace_bytes, hipStream_t s, const char* who) {
  const int es = dtype_size(dtype);
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
  a.q_heads = q_heads;
  a.group = q_heads / kv_heads;
  a.head_dim = head_dim;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.window = window;
  a.table_width = table_width;
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)head_dim));
  // Pages per split: at least kSplitTokens tokens; without a workspace every
  // row is a single split (pages can never exceed the table width).
  a.min_bps = workspace != nullptr ? std::max(1, kSplitTokens / block_size)
                                   : std::max(1, table_width);

  // Largest split count any row of this table width can need: the grid is a
  // function of shapes only (graph capture), never of device lengths.
  const int max_pages = std::max(1, table_width);
  const int gx = std::max(1, std::min(kMaxSplits, ceil_div(max_pages, a.min_bps)));
  for (int64_t first = 0; first < rows; first += 65535) {
    a.row_base = first;
    const unsigned count = (unsigned)std::min<int64_t>(rows - first, 65535);
    bool ok = false;
    dim3 grid((unsigned)gx, (unsigned)q_heads, count);
    switch (dtype) {
      case VRH_DTYPE_F32: ok = launch_decode<float>(vec, lpt, grid, s, a); break;
      case VRH_DTYPE_F16: ok = launch_decode<f16_t>(vec, lpt, grid, s, a); break;
      case VRH_DTYPE_BF16: ok = launch_decode<bf16_t>(vec, lpt, grid, s, a); break;
    }
    VRH_CHECK_ARG(ok, "%s: no kernel for vec=%d lanes=%d", who, vec, lpt);
    if (gx == 1) continue;  // every row is a single split: output already written
    dim3 mgrid((unsigned)q_heads, count);
    switch (dtype) {
      case VRH_DTYPE_F32:
        hipLaunchKernelGGL(paged_decode_merge_kernel<float>, mgrid, dim3(64), 0, s, a);
        break;
      case VRH_DTYPE_F16:
        hipLaunchKernelGGL(paged_decode_merge_kernel<f16_t>, mgrid, dim3(64), 0, s, a);
        break;
      case VRH_DTYPE_BF16:
        hipLaunchKernelGGL(paged_decode_merge_kernel<bf16_t>, mgrid, dim3(64), 0, s, a);
        break;
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
                         nullptr, 0, rows, q_heads, kv_heads, head_dim, block_size, table_width,
                         table_stride, q_row_stride, q_head_stride, out_row_stride,
                         out_head_stride, k_block_stride, k_token_stride, k_head_stride,
                         v_block_stride, v_token_stride, v_head_stride, window, workspace,
                         workspace_bytes, (hipStream_t)stream, "vrh_paged_decode");
}
