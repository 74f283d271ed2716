// Packed causal (WCPB chunked) prefill over paged K/V, MFMA on gfx950.
//
// Reference semantics: kernels/triton_attention.py:205-366. Sequence s owns
// query rows [cu[s], cu[s+1]) and keys [0, n_s) through block_tables[s]; its
// query i sits at position n_s - q_s + i (bottom-right alignment) and attends
// keys at positions <= that. fp32 online softmax; P is rounded to the storage
// dtype before the PV product (as the reference's `weights.to(values.dtype)`).
//
// MFMA path (bf16/f16, head_dim a multiple of 32 up to 224, LDS-bound):
//  * Workgroup = 4 waves = 64 query rows of one (sequence, q head); each wave
//    owns 16 queries. K/V tiles of 64 keys are staged in LDS once per
//    workgroup and shared by the 4 waves; the next tile is prefetched into
//    registers while the current one is consumed.
//  * S^T = K Q^T with v_mfma_f32_16x16x32_{bf16,f16}: A = K rows from LDS
//    (16-byte reads), B = Q^T held in registers for the whole kernel.
//    Output lane l holds query l % 16 and keys 4 * (l / 16) + j, j < 4.
//  * O^T = V^T P^T: the S^T accumulator of a lane is already a P^T B-operand
//    (same query column, keys in the lane's k-slots), so P never goes through
//    LDS. V is stored transposed in LDS ([d][key]) when the tile is staged; A
//    reads are two 8-byte reads whose keys match the P^T k-slots. Only the
//    pairing of A and B k-slots matters, not the hardware's k order.
//  * Per-query running max is reduced over the 4 lane groups each tile; the
//    running sum stays a per-lane partial until the end.
// Other dtypes / head dims (f32 reference checks, odd dims) run the decode
// kernel over the expanded rows: query i of sequence s is a decode row with
// length n_s - q_s + i + 1 (the per-row formulation the reference tests use).
#include <algorithm>

#include "common.h"

int vrh_decode_rows(int dtype, void* out, const void* q, const void* key_cache,
                    const void* value_cache, const int32_t* block_tables,
                    const int32_t* context_lengths, const int32_t* cu_q, int32_t num_seqs,
                    int32_t expand_e, int64_t rows, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                    int32_t block_size, int32_t table_width, int64_t table_stride,
                    int64_t q_row_stride, int64_t q_head_stride, int64_t out_row_stride,
                    int64_t out_head_stride, int64_t k_block_stride, int64_t k_token_stride,
                    int64_t k_head_stride, int64_t v_block_stride, int64_t v_token_stride,
                    int64_t v_head_stride, int32_t window, void* workspace,
                    size_t workspace_bytes, hipStream_t s, const char* who);

namespace vrh {
namespace {

constexpr int kBM = 64;  // queries per workgroup (16 per wave)
constexpr int kBN = 64;  // keys per tile

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

template <typename T>
struct Mfma;
template <>
struct Mfma<bf16_t> {
  __device__ static f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<f16_t> {
  __device__ static f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

__device__ __forceinline__ uint32_t bits16(bf16_t x) { return x.bits; }
__device__ __forceinline__ uint32_t bits16(f16_t x) {
  return (uint32_t)__builtin_bit_cast(uint16_t, x);
}
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return bits16(from_f32<T>(lo)) | (bits16(from_f32<T>(hi)) << 16);
}

struct PrefillArgs {
  void* out;
  const void* q;
  const void* k;
  const void* v;
  const int32_t* tables;
  const int32_t* lengths;
  const int32_t* cu;
  int64_t q_token, q_head, o_token, o_head;
  int64_t k_block, k_token, k_head;
  int64_t v_block, v_token, v_head;
  int64_t table_stride;
  int64_t seq_base;
  int32_t group, block_size, bs_shift, table_width;
  int32_t skip_q;  // sequences with q_len <= skip_q are left to the decode kernel
  float scale_log2;
};

// LDS row pitches (elements): +8 / +4 padding breaks bank aliasing of the
// 16-lane row reads.
template <int D>
struct Lds {
  static constexpr int kPitch = D + 8;     // K tile [kBN][kPitch]
  static constexpr int vPitch = kBN + 4;   // V^T tile [D][vPitch]
  static constexpr int kElems = kBN * kPitch;
  static constexpr int vElems = D * vPitch;
};

template <typename T, int D>
__global__ __launch_bounds__(256) void paged_prefill_kernel(PrefillArgs a) {
  constexpr int DC = D / 32;         // 32-wide d chunks (QK^T k-steps)
  constexpr int DT = D / 16;         // 16-row d tiles of O^T
  constexpr int KCH = D / 8;         // 16-byte chunks per K row
  constexpr int KLOADS = kBN * KCH / 256;   // K tile vectors per thread
  constexpr int VUNITS = (kBN / 4) * KCH;   // (4 keys x 8 dims) units per V tile
  constexpr int VLOADS = (VUNITS + 255) / 256;
  static_assert(D % 32 == 0 && D <= 256, "head_dim");
  static_assert(kBN * KCH % 256 == 0, "K tile split");

  __shared__ __attribute__((aligned(16))) uint16_t ks[Lds<D>::kElems];
  __shared__ __attribute__((aligned(16))) uint16_t vts[Lds<D>::vElems];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;  // query column within the wave's 16
  const int grp = lane >> 4;  // lane group 0..3
  const int64_t seq = a.seq_base + blockIdx.z;
  const int head = blockIdx.y;
  const int kvh = head / a.group;
  const int q_begin = a.cu[seq];
  const int q_len = a.cu[seq + 1] - q_begin;
  if ((int)blockIdx.x * kBM >= q_len || q_len <= a.skip_q) return;
  int n = a.lengths[seq];
  {
    const int64_t cap = (int64_t)a.table_width * a.block_size;
    n = n < 0 ? 0 : ((int64_t)n > cap ? (int)cap : n);
  }
  const int prefix = n - q_len;
  const int qi = blockIdx.x * kBM + wave * 16 + col;  // this lane's query
  const bool q_ok = qi < q_len;
  const int qpos = prefix + qi;
  const int end = max(0, min(n, prefix + ((int)blockIdx.x + 1) * kBM));
  const int32_t* table = a.tables + seq * a.table_stride;

  // Q^T B-operands: lane holds query `col`, dims 32c + 8*grp .. +8.
  u32x4 qop[DC];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)(q_begin + qi) * a.q_token +
                  head * a.q_head + 8 * grp;
#pragma unroll
    for (int c = 0; c < DC; ++c)
      qop[c] = q_ok ? *reinterpret_cast<const u32x4*>(qp + 32 * c) : u32x4{0, 0, 0, 0};
  }

  f32x4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY;  // running max of this lane's query (log2 domain)
  float lsum = 0.f;     // partial sum over this lane's key slots

  const T* kg = reinterpret_cast<const T*>(a.k) + kvh * a.k_head;
  const T* vg = reinterpret_cast<const T*>(a.v) + kvh * a.v_head;

  u32x4 kreg[KLOADS];
  u32x4 vreg[VLOADS][4];
  // Page ids of the keys this thread stages, fetched one tile ahead of the
  // K/V loads so those never wait on a page-table read.
  int32_t kpg[KLOADS];
  int32_t vpg[VLOADS][4];
  auto split_pos = [&](int pos, int& page, int& off) {
    if (a.bs_shift >= 0) {
      page = pos >> a.bs_shift;
      off = pos & (a.block_size - 1);
    } else {
      page = pos / a.block_size;
      off = pos - page * a.block_size;
    }
  };
  auto fetch_pages = [&](int t0) {
#pragma unroll
    for (int r = 0; r < KLOADS; ++r) {
      const int key = (tid + 256 * r) / KCH;
      const int pos = t0 + key;
      int page, off;
      split_pos(pos, page, off);
      kpg[r] = pos < end ? table[page] : 0;
    }
#pragma unroll
    for (int r = 0; r < VLOADS; ++r) {
      const int kq = (tid + 256 * r) / KCH;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int pos = t0 + 4 * kq + j;
        int page, off;
        split_pos(pos, page, off);
        vpg[r][j] = (tid + 256 * r < VUNITS && pos < end) ? table[page] : 0;
      }
    }
  };
  // Global -> registers for the tile starting at key t0 (zeros past `end`).
  auto fetch = [&](int t0) {
#pragma unroll
    for (int r = 0; r < KLOADS; ++r) {
      const int c = tid + 256 * r;
      const int key = c / KCH, dc = c % KCH;
      const int pos = t0 + key;
      if (pos < end) {
        int page, off;
        split_pos(pos, page, off);
        kreg[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            kg + (int64_t)kpg[r] * a.k_block + off * a.k_token + dc * 8));
      } else {
        kreg[r] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int r = 0; r < VLOADS; ++r) {
      const int u = tid + 256 * r;
      const int kq = u / KCH, dc = u % KCH;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int pos = t0 + 4 * kq + j;
        if (u < VUNITS && pos < end) {
          int page, off;
          split_pos(pos, page, off);
          vreg[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
              vg + (int64_t)vpg[r][j] * a.v_block + off * a.v_token + dc * 8));
        } else {
          vreg[r][j] = u32x4{0, 0, 0, 0};
        }
      }
    }
  };
  // Registers -> LDS: K row-major, V transposed to [d][key].
  auto stash = [&]() {
#pragma unroll
    for (int r = 0; r < KLOADS; ++r) {
      const int c = tid + 256 * r;
      const int key = c / KCH, dc = c % KCH;
      *reinterpret_cast<u32x4*>(&ks[key * Lds<D>::kPitch + dc * 8]) = kreg[r];
    }
#pragma unroll
    for (int r = 0; r < VLOADS; ++r) {
      const int u = tid + 256 * r;
      if (u < VUNITS) {
        const int kq = u / KCH, dc = u % KCH;
#pragma unroll
        for (int e = 0; e < 8; ++e) {  // dim dc*8 + e, keys 4kq .. 4kq+3
          const int w = e >> 1, sh = (e & 1) * 16;
          const uint32_t k0 = (vreg[r][0][w] >> sh) & 0xffffu;
          const uint32_t k1 = (vreg[r][1][w] >> sh) & 0xffffu;
          const uint32_t k2 = (vreg[r][2][w] >> sh) & 0xffffu;
          const uint32_t k3 = (vreg[r][3][w] >> sh) & 0xffffu;
          *reinterpret_cast<u32x2*>(&vts[(dc * 8 + e) * Lds<D>::vPitch + 4 * kq]) =
              u32x2{k0 | (k1 << 16), k2 | (k3 << 16)};
        }
      }
    }
  };

  if (end > 0) {
    fetch_pages(0);
    fetch(0);
    if (kBN < end) fetch_pages(kBN);
  }
  for (int t0 = 0; t0 < end; t0 += kBN) {
    __syncthreads();  // previous tile fully consumed
    stash();
    __syncthreads();
    if (t0 + kBN < end) {
      fetch(t0 + kBN);  // in flight while we compute
      if (t0 + 2 * kBN < end) fetch_pages(t0 + 2 * kBN);
    }

    // S^T tiles: st[kt] holds keys t0 + 16kt + 4grp + j for query `col`.
    f32x4 st[kBN / 16];
#pragma unroll
    for (int kt = 0; kt < kBN / 16; ++kt) {
      f32x4 c4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const u32x4 kop =
            *reinterpret_cast<const u32x4*>(&ks[(16 * kt + col) * Lds<D>::kPitch + 32 * c + 8 * grp]);
        c4 = Mfma<T>::run(kop, qop[c], c4);
      }
      st[kt] = c4;
    }
    // Scale, mask (causal + tile end), running max over the 4 lane groups.
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < kBN / 16; ++kt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kpos = t0 + 16 * kt + 4 * grp + j;
        const bool vis = q_ok && kpos < end && kpos <= qpos;
        const float sv = vis ? st[kt][j] * a.scale_log2 : -INFINITY;
        st[kt][j] = sv;
        mx = fmaxf(mx, sv);
      }
    }
    mx = fmaxf(mx, shfl_xor_f32(mx, 16));
    mx = fmaxf(mx, shfl_xor_f32(mx, 32));
    const float mnew = fmaxf(m, mx);
    const float safe = mnew == -INFINITY ? 0.f : mnew;
    const float corr = exp2f(m - safe);
    lsum *= corr;
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] *= corr;
    // P^T operands per 32-key chunk: slots 0..3 from tile 2kc, 4..7 from 2kc+1.
    u32x4 pop[kBN / 32];
#pragma unroll
    for (int kc = 0; kc < kBN / 32; ++kc) {
      float p[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p[j] = exp2f(st[2 * kc][j] - safe);
        p[4 + j] = exp2f(st[2 * kc + 1][j] - safe);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) lsum += p[j];
      pop[kc] = u32x4{pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3]), pack2<T>(p[4], p[5]),
                      pack2<T>(p[6], p[7])};
    }
    m = mnew;
    // O^T[d, q] += V^T[d, keys] P^T[keys, q]
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const uint16_t* vrow = &vts[(16 * t + col) * Lds<D>::vPitch];
#pragma unroll
      for (int kc = 0; kc < kBN / 32; ++kc) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow + 32 * kc + 4 * grp);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 32 * kc + 16 + 4 * grp);
        acc[t] = Mfma<T>::run(u32x4{lo[0], lo[1], hi[0], hi[1]}, pop[kc], acc[t]);
      }
    }
  }

  lsum += shfl_xor_f32(lsum, 16);
  lsum += shfl_xor_f32(lsum, 32);
  if (!q_ok) return;
  const float inv = 1.f / fmaxf(lsum, 1e-30f);
  T* op = reinterpret_cast<T*>(a.out) + (int64_t)(q_begin + qi) * a.o_token + head * a.o_head;
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    const int d = 16 * t + 4 * grp;
    *reinterpret_cast<u32x2*>(op + d) =
        u32x2{pack2<T>(acc[t][0] * inv, acc[t][1] * inv), pack2<T>(acc[t][2] * inv, acc[t][3] * inv)};
  }
}

template <typename T>
bool launch_prefill(int d, dim3 grid, hipStream_t s, const PrefillArgs& a) {
  switch (d) {
#define VRH_D(DV)                                                                    \
  case DV:                                                                           \
    hipLaunchKernelGGL((paged_prefill_kernel<T, DV>), grid, dim3(256), 0, s, a); \
    return true;
    VRH_D(32)
    VRH_D(64)
    VRH_D(96)
    VRH_D(128)
    VRH_D(160)
    VRH_D(192)
    VRH_D(224)
#undef VRH_D
    default: return false;
  }
}

}  // namespace
}  // namespace vrh

using namespace vrh;

// Sequences with at most this many queries (decode rows riding in a packed
// batch) run through the split-KV decode kernel instead of 64-query MFMA tiles.
constexpr int kDecodeQ = 1;

extern "C" size_t vrh_paged_prefill_workspace_bytes(int64_t num_seqs, int32_t q_heads,
                                                    int32_t head_dim) {
  return vrh_paged_decode_workspace_bytes(num_seqs * kDecodeQ, q_heads, head_dim);
}

extern "C" int vrh_paged_prefill(int dtype, void* out, const void* q, const void* key_cache,
                                 const void* value_cache, const int32_t* block_tables,
                                 const int32_t* context_lengths, const int32_t* cu_seqlens_q,
                                 int64_t num_seqs, int64_t total_q, int32_t max_seqlen_q,
                                 int32_t q_heads, int32_t kv_heads, int32_t head_dim,
                                 int32_t block_size, int32_t table_width, int64_t table_stride,
                                 int64_t q_token_stride, int64_t q_head_stride,
                                 int64_t out_token_stride, int64_t out_head_stride,
                                 int64_t k_block_stride, int64_t k_token_stride,
                                 int64_t k_head_stride, int64_t v_block_stride,
                                 int64_t v_token_stride, int64_t v_head_stride, void* workspace,
                                 size_t workspace_bytes, vrh_stream_t stream) {
  VRH_CHECK_ARG(num_seqs >= 0 && total_q >= 0 && max_seqlen_q >= 0,
                "vrh_paged_prefill: bad sizes");
  VRH_CHECK_ARG(q_heads >= 1 && kv_heads >= 1 && q_heads % kv_heads == 0,
                "vrh_paged_prefill: query heads must be a positive multiple of KV heads");
  VRH_CHECK_ARG(num_seqs < (1ll << 31) / kDecodeQ, "vrh_paged_prefill: too many sequences");
  if (num_seqs == 0 || total_q == 0) return VRH_OK;
  VRH_CHECK_ARG(out && q && key_cache && value_cache && block_tables && context_lengths &&
                    cu_seqlens_q,
                "vrh_paged_prefill: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const bool half = dtype == VRH_DTYPE_BF16 || dtype == VRH_DTYPE_F16;
  bool mfma = half && head_dim % 32 == 0 && head_dim <= 224 && block_size >= 1 &&
              q_token_stride % 8 == 0 && q_head_stride % 8 == 0 && out_token_stride % 4 == 0 &&
              out_head_stride % 4 == 0 && k_block_stride % 8 == 0 && k_token_stride % 8 == 0 &&
              k_head_stride % 8 == 0 && v_block_stride % 8 == 0 && v_token_stride % 8 == 0 &&
              v_head_stride % 8 == 0;
  for (const void* p : {(const void*)out, q, key_cache, value_cache}) mfma = mfma && ((uintptr_t)p % 16 == 0);
  if (!mfma) {
    return vrh_decode_rows(dtype, out, q, key_cache, value_cache, block_tables, context_lengths,
                           cu_seqlens_q, (int32_t)num_seqs, 0, total_q, q_heads, kv_heads,
                           head_dim, block_size, table_width, table_stride, q_token_stride,
                           q_head_stride, out_token_stride, out_head_stride, k_block_stride,
                           k_token_stride, k_head_stride, v_block_stride, v_token_stride,
                           v_head_stride, 0, nullptr, 0, s, "vrh_paged_prefill");
  }
  VRH_CHECK_ARG(max_seqlen_q >= 1, "vrh_paged_prefill: max_seqlen_q must be positive");
  VRH_CHECK_ARG(q_heads <= 65535, "vrh_paged_prefill: too many heads");
  const bool route_decode =
      workspace != nullptr &&
      workspace_bytes >= vrh_paged_prefill_workspace_bytes(num_seqs, q_heads, head_dim);
  PrefillArgs a;
  a.out = out;
  a.q = q;
  a.k = key_cache;
  a.v = value_cache;
  a.tables = block_tables;
  a.lengths = context_lengths;
  a.cu = cu_seqlens_q;
  a.q_token = q_token_stride;
  a.q_head = q_head_stride;
  a.o_token = out_token_stride;
  a.o_head = out_head_stride;
  a.k_block = k_block_stride;
  a.k_token = k_token_stride;
  a.k_head = k_head_stride;
  a.v_block = v_block_stride;
  a.v_token = v_token_stride;
  a.v_head = v_head_stride;
  a.table_stride = table_stride;
  a.group = q_heads / kv_heads;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.table_width = table_width;
  a.skip_q = route_decode ? kDecodeQ : 0;
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)head_dim));
  const unsigned qblocks = (unsigned)ceil_div(max_seqlen_q, kBM);
  for (int64_t first = 0; first < num_seqs; first += 65535) {
    a.seq_base = first;
    const unsigned count = (unsigned)std::min<int64_t>(num_seqs - first, 65535);
    dim3 grid(qblocks, (unsigned)q_heads, count);
    const bool ok = dtype == VRH_DTYPE_BF16 ? launch_prefill<bf16_t>(head_dim, grid, s, a)
                                            : launch_prefill<f16_t>(head_dim, grid, s, a);
    VRH_CHECK_ARG(ok, "vrh_paged_prefill: no kernel for head_dim %d", head_dim);
  }
  if (route_decode) {
    // Decode rows of the packed batch: split-KV single-query kernel.
    const int rc = vrh_decode_rows(
        dtype, out, q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q,
        (int32_t)num_seqs, kDecodeQ, num_seqs * kDecodeQ, q_heads, kv_heads, head_dim,
        block_size, table_width, table_stride, q_token_stride, q_head_stride, out_token_stride,
        out_head_stride, k_block_stride, k_token_stride, k_head_stride, v_block_stride,
        v_token_stride, v_head_stride, 0, workspace, workspace_bytes, s, "vrh_paged_prefill");
    if (rc != VRH_OK) return rc;
  }
  VRH_RETURN_LAUNCH("vrh_paged_prefill");
}
