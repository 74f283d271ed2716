// Packed causal (WCPB chunked) prefill over paged K/V, MFMA on gfx950.
//
// Reference semantics: kernels/triton_attention.py:205-366. Sequence s owns
// query rows [cu[s], cu[s+1]) and keys [0, n_s) through block_tables[s]; its
// query i sits at position n_s - q_s + i (bottom-right alignment) and attends
// keys at positions <= that. fp32 online softmax; P is rounded to the storage
// dtype before the PV product (as the reference's `weights.to(values.dtype)`).
//
// MFMA path (bf16/f16, head_dim a multiple of 32 up to 128):
//  * Workgroup = 4 waves = 128 query rows of one (sequence, q head); each wave
//    owns 32 queries. K/V arrive in 32-key sub-blocks staged into LDS (three
//    stages, loaded straight into LDS two sub-blocks ahead) and shared by
//    the 4 waves; one barrier per sub-block.
//  * Three workgroups per CU (three waves per SIMD, at most 168 VGPRs): a
//    wave runs QK^T, softmax and PV of one sub-block in order, reading each
//    MFMA operand from LDS one MFMA ahead of its use, and the SIMD's other
//    two waves fill the MFMA and VALU pipes while it waits.
//  * S^T = K Q^T with v_mfma_f32_32x32x16_{bf16,f16}: A = K rows from LDS
//    (16-byte reads), B = Q^T held in registers for the whole kernel.
//    Output lane l holds query l % 32 and keys 8 * (j / 4) + 4 * (l / 32) + j % 4.
//  * O^T = V^T P^T: the S^T accumulator of a lane is already a P^T B-operand
//    (same query column, keys in the lane's k-slots), so P never goes through
//    LDS. V stays row-major in LDS; the V^T A-operand comes from two
//    ds_read_b64_tr_b16 transposed reads whose keys match the P^T k-slots.
//    Only the pairing of A and B k-slots matters, not the hardware's k order.
//  * Per-query running max is reduced over the lane pair (l, l ^ 32) each
//    sub-block; the running sum stays a per-lane partial until the end.
// Other dtypes / head dims (f32 reference checks, odd dims) run the decode
// kernel over the expanded rows: query i of sequence s is a decode row with
// length n_s - q_s + i + 1 (the per-row formulation the reference tests use).
#include <algorithm>
#include <type_traits>

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

constexpr int kWaves = 4;                  // waves per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kWQ = 32;                    // queries per wave
constexpr int kBM = kWQ * kWaves;          // queries per workgroup
constexpr int kSB = 32;                    // keys per sub-block (one pipeline step)
constexpr int kStages = 3;                 // LDS stages: one sub-block each
constexpr int kTableSeg = 512;             // page ids staged in LDS at a time

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

// 32x32x16 MFMA: A lane l = row l % 32 with k-slots 8 * (l / 32) + i, B lane
// l = column l % 32 with the same k-slots; D lane l = column l % 32, element j
// = row 8 * (j / 4) + 4 * (l / 32) + j % 4.
template <typename T>
struct Mfma;
template <>
struct Mfma<bf16_t> {
  __device__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<f16_t> {
  __device__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

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
  int64_t num_seqs;
  int32_t qblocks, kv_heads;
  int32_t group, block_size, bs_shift, table_width;
  int32_t skip_q;  // sequences with q_len <= skip_q are left to the decode kernel
  int32_t uniform_pages;  // block size a power-of-two multiple of 256 / (16-byte chunks per row)
  int32_t same_kv32;      // K and V block/token strides equal and below 2^31
  const int32_t* order;   // sequences in dispatch order (longest first), or null
  int32_t rank_in_kernel; // num_seqs <= 64: each wave ranks the sequences itself
  float scale_log2;
};

// LDS tiles (one 32-key sub-block of K and of V per stage), both row-major
// [key][d] without padding: each 16-byte staging store of a wave fills 64
// consecutive 16-byte slots. Bank conflicts are removed by an XOR swizzle of
// the 16-byte chunk index inside each row instead:
// chunk c of row r is stored at slot c ^ swizzle(r). For 256-byte rows
// (D = 128) swizzle(r) = ((r & 3) << 2) ^ ((r >> 2) & 3) serves both readers
// at the full 256 B/clk: the K operand read (32 rows, one chunk each) and the
// transposed V read (8 rows x 4 chunks). Narrower rows pack 256 / (16 * KCH)
// rows into one bank window and swizzle on the window index instead.
template <int D>
struct Lds {
  static constexpr int KCH = D / 8;  // 16-byte chunks per row
  static constexpr int kElems = kSB * D;  // one sub-block of K (or V)
  __device__ static int swizzle(int row) {
    if constexpr (KCH == 16) return ((row & 3) << 2) ^ ((row >> 2) & 3);
    else if constexpr (KCH == 8) return (((row >> 1) & 1) << 2) ^ ((row >> 2) & 3);
    else if constexpr (KCH == 4) return (row >> 2) & 3;
    else if constexpr (KCH % 8 == 0) return row & 7;
    else return row & 3;  // KCH = 12, 20, 28: XOR stays inside 4-chunk groups
  }
  // Element offset of dim `d` of key row `row` (d % 8 kept inside its chunk).
  __device__ static int at(int row, int d) {
    return row * D + (((d >> 3) ^ swizzle(row)) << 3) + (d & 7);
  }
};

// ds_read_b64_tr_b16: within each 16-lane group, lane j receives element j % 4
// of the 8-byte chunks addressed by lanes 4i + j / 4, i = 0..3 (element i of
// the result). Lanes 4i + s that address row (key) r0 + i, dims d0 + 4s .. +3
// therefore give lane j dims d0 + j of keys r0 .. r0 + 3.
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (v4s __attribute__((address_space(3)))*)(const_cast<uint16_t*>(p)));
  return __builtin_bit_cast(u32x2, r);
}

// Three workgroups per CU, three waves per SIMD.
constexpr int kWgPerCu = 3;
constexpr int kWavesPerEu = kWgPerCu * kWaves / 4;

// Page addressing modes: kDiv (any block size), kShift (power of two).
enum PageMode { kDiv = 0, kShift = 1 };

template <typename T, int D, int MODE>
__global__ __launch_bounds__(kThreads, kWgPerCu)
__attribute__((amdgpu_waves_per_eu(kWavesPerEu, kWavesPerEu))) void paged_prefill_kernel(PrefillArgs a) {
  constexpr int DC = D / 16;                   // 16-wide d chunks (QK^T k-steps)
  constexpr int DB = D / 32;                   // 32-row d blocks of O^T
  constexpr int KCH = D / 8;                   // 16-byte chunks per key row
  constexpr int SB_INST = kSB * KCH / 64;      // 16-byte wave stores per sub-block (K or V)
  constexpr int NI = (SB_INST + kWaves - 1) / kWaves;  // per wave (the last may be idle)
  static_assert(D % 32 == 0 && D <= 128, "head_dim");
  using L = Lds<D>;

  __shared__ __attribute__((aligned(16))) uint16_t ks[kStages][L::kElems];
  __shared__ __attribute__((aligned(16))) uint16_t vs[kStages][L::kElems];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;  // query column of this lane
  const int half = lane >> 5; // k-slot half (0 or 1)
  // XCD-aware order: workgroup ids are dealt round-robin to the 8 XCDs (id L
  // runs on XCD L % 8). A group = one (sequence, kv head); its work items --
  // every query block of every q head reading that K/V -- all go to XCD
  // group % 8, back to back, so their K/V tiles are shared in that XCD's L2.
  // Within a group the longest (last) query blocks run first.
  const int per_group = a.group * a.qblocks;
  const int64_t slot = blockIdx.x / 8;
  const int64_t g = (slot / per_group) * 8 + blockIdx.x % 8;
  if (g >= a.num_seqs * a.kv_heads) return;
  const int r_item = (int)(slot % per_group);
  const int head = (int)(g % a.kv_heads) * a.group + r_item / a.qblocks;
  const int qb = a.qblocks - 1 - r_item % a.qblocks;
  const int kvh = head / a.group;
  const int64_t cap = (int64_t)a.table_width * a.block_size;
  int64_t seq;
  int q_begin, q_len, n;
  if (a.rank_in_kernel) {
    // Up to 64 sequences: every wave ranks them itself (one lane per
    // sequence, the same longest-first stable order as prefill_order_kernel)
    // and takes the sequence of rank g / kv_heads, without a separate launch.
    const int s = lane;
    int c0 = 0, c1 = 0, len = 0, key = INT32_MIN;
    if (s < a.num_seqs) {
      c0 = a.cu[s];
      c1 = a.cu[s + 1];
      len = a.lengths[s];
      key = c1 - c0 <= a.skip_q ? -1 : (int)(len < 0 ? 0 : ((int64_t)len > cap ? cap : len));
    }
    int rank = 0;
#pragma unroll
    for (int j = 0; j < 64; ++j) {
      const int other = __builtin_amdgcn_readlane(key, j);
      rank += (other > key) || (other == key && j < s);
    }
    const uint64_t hit = __ballot(rank == (int)(g / a.kv_heads) && s < a.num_seqs);
    const int pick = __builtin_ffsll((long long)hit) - 1;
    seq = pick;
    q_begin = __builtin_amdgcn_readlane(c0, pick);
    q_len = __builtin_amdgcn_readlane(c1, pick) - q_begin;
    n = __builtin_amdgcn_readlane(len, pick);
  } else {
    seq = a.order ? a.order[g / a.kv_heads] : g / a.kv_heads;
    q_begin = a.cu[seq];
    q_len = a.cu[seq + 1] - q_begin;
    n = a.lengths[seq];
  }
  if (qb * kBM >= q_len || q_len <= a.skip_q) return;
  n = n < 0 ? 0 : ((int64_t)n > cap ? (int)cap : n);
  const int prefix = n - q_len;
  const int qi0 = qb * kBM + wave * kWQ;        // this wave's first query
  const int qi = qi0 + col;                     // this lane's query
  const bool q_ok = qi < q_len;
  const int qpos = prefix + qi;
  const int wave_qpos0 = prefix + qi0;
  const int end = max(0, min(n, prefix + (qb + 1) * kBM));
  const int nsub = (end + kSB - 1) / kSB;       // sub-blocks staged by the workgroup
  // Sub-blocks this wave computes: keys up to its last query's position.
  const int nsub_w = qi0 >= q_len ? 0 : (max(0, min(end, wave_qpos0 + kWQ)) + kSB - 1) / kSB;
  const int32_t* table = a.tables + seq * a.table_stride;

  // Q^T B-operands: lane holds query `col`, dims 16c + 8*half .. +8.
  u32x4 qop[DC];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + (int64_t)(q_begin + (q_ok ? qi : 0)) * a.q_token +
                  head * a.q_head + 8 * half;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qp + 16 * c);
      qop[c] = q_ok ? v : u32x4{0, 0, 0, 0};
    }
  }

  f32x16 acc[DB];
#pragma unroll
  for (int t = 0; t < DB; ++t) acc[t] = f32x16{};
  // Reference max of this lane's query in the log2 domain; finite so that
  // fully masked scores give exp2(-inf) = 0.
  float m = -1e30f;
  float lsum = 0.f;     // partial sum over this lane's key slots

  const T* kg = reinterpret_cast<const T*>(a.k) + kvh * a.k_head;
  const T* vg = reinterpret_cast<const T*>(a.v) + kvh * a.v_head;

  // A 512-entry segment of the page table is staged in LDS. A page id
  // fetched with a vector load would make every later K/V load wait for all
  // earlier ones (vmcnt retires in order), so the per-key lookups read LDS;
  // the segment is refilled (all waves, between barriers) when a sub-block's
  // pages run past it.
  __shared__ int32_t tbl_lds[kTableSeg];
  int tbl_base = 0;
  auto load_table = [&](int base) {
    __syncthreads();
    for (int i = tid; i < kTableSeg; i += kThreads)
      tbl_lds[i] = base + i < a.table_width ? table[base + i] : 0;
    __syncthreads();
    tbl_base = base;
  };
  auto page_of = [&](int pos) {
    if constexpr (MODE == kDiv) return pos / a.block_size;
    else return pos >> a.bs_shift;
  };
  load_table(0);

  // Sub-block `j` of K/V goes from the pages straight into an LDS stage.
  // Staging instruction r of this wave fills slots 64 * (wave + 4r) .. + 63 of
  // the sub-block: slot v holds chunk (v % KCH) ^ swizzle(row) of key row
  // v / KCH. Branch-free: keys past `end` re-read key end - 1 (real data);
  // the softmax masks them.
  // With KCH a power of two a lane keeps its chunk and its row advances by
  // S = 64 * kWaves / KCH per instruction, so the swizzled chunk offset (the
  // swizzle depends on row % 16, and S is a multiple of 16) is a per-lane
  // constant. One instruction covers the IR = 64 / KCH consecutive rows
  // starting at row k0 + IR * inst; when the block size is a multiple of IR
  // they share a page, so a full sub-block needs one (wave-uniform) page-id
  // read per instruction and the lane adds its row within the instruction.
  constexpr bool kPow2 = (KCH & (KCH - 1)) == 0;
  constexpr int S = 64 * kWaves / KCH;
  constexpr int IR = 64 / KCH;
  static_assert(!kPow2 || S % 16 == 0, "swizzle period");
  const int lane_row = (64 * wave + lane) / KCH;
  const int lane_dof = kPow2 ? (((64 * wave + lane) % KCH) ^ L::swizzle(lane_row)) * 8 : 0;
  const int lane_in = lane / KCH;  // row within one instruction's IR rows
  const T* lane_k = kg + (int64_t)lane_row * a.k_token + lane_dof;
  const T* lane_v = vg + (int64_t)lane_row * a.v_token + lane_dof;
  const T* lane_k1 = kg + (int64_t)lane_in * a.k_token + lane_dof;
  const T* lane_v1 = vg + (int64_t)lane_in * a.v_token + lane_dof;
  // Byte offset of this lane's 16 bytes within one staging instruction's rows
  // (same for K and V when their strides match); 32-bit when it fits.
  const int64_t lane_koff64 = ((int64_t)lane_in * a.k_token + lane_dof) * (int64_t)sizeof(T);
  const bool lane_off32 = (int64_t)(IR - 1) * a.k_token * (int64_t)sizeof(T) + 2 * D < (1ll << 31);
  const uint32_t lane_koff = (uint32_t)lane_koff64;
  // Addresses of sub-block j's K and V vectors for this wave's staging
  // instructions r = 0 .. NI - 1, handed to `sink(r, k_ptr, v_ptr)`.
  auto gather_to = [&](int j, auto&& sink) {
    const int k0 = j * kSB;
    {
      const int last_page = page_of(min(k0 + kSB, end) - 1);
      if (last_page >= tbl_base + kTableSeg) load_table(page_of(k0));
    }
    auto pad = [&](int inst) { return SB_INST % kWaves != 0 && inst >= SB_INST; };
    if (kPow2 && a.uniform_pages && a.same_kv32 && k0 + kSB <= end) {
      // K and V share block / token strides below 2^31 elements: one 32 x 32
      // -> 64-bit scalar product per instruction addresses both.
#pragma unroll
      for (int r = 0; r < NI; ++r) {
        const int inst = wave + kWaves * r;
        if (pad(inst)) continue;
        const int pb = k0 + IR * inst;  // first row of this instruction
        const uint32_t page = __builtin_amdgcn_readfirstlane(tbl_lds[(pb >> a.bs_shift) - tbl_base]);
        const uint32_t row_off = __builtin_amdgcn_readfirstlane(pb & (a.block_size - 1));
        const uint64_t off = (uint64_t)page * (uint32_t)a.k_block +
                             (uint64_t)row_off * (uint32_t)a.k_token;
        sink(r, lane_k1 + off, lane_v1 + off);
      }
      return;
    }
    if (kPow2 && a.uniform_pages && k0 + kSB <= end) {
#pragma unroll
      for (int r = 0; r < NI; ++r) {
        const int inst = wave + kWaves * r;
        if (pad(inst)) continue;
        const int pb = k0 + IR * inst;  // first row of this instruction
        const int pg = pb >> a.bs_shift;
        const int64_t page = __builtin_amdgcn_readfirstlane(tbl_lds[pg - tbl_base]);
        const int64_t row_off = __builtin_amdgcn_readfirstlane(pb & (a.block_size - 1));
        sink(r, lane_k1 + (page * a.k_block + row_off * a.k_token),
             lane_v1 + (page * a.v_block + row_off * a.v_token));
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < NI; ++r) {
      const int inst = wave + kWaves * r;
      if (pad(inst)) continue;
      const int v = 64 * inst + lane;
      const int row = kPow2 ? lane_row + r * S : v / KCH;
      const int dof = kPow2 ? 0 : ((v % KCH) ^ L::swizzle(row)) * 8;
      const int pos = min(k0 + row, end - 1);
      const int pg = page_of(pos);
      const int64_t page = tbl_lds[pg - tbl_base];
      const int64_t toks = pos - pg * a.block_size - (kPow2 ? lane_row : 0);
      sink(r, (kPow2 ? lane_k : kg) + page * a.k_block + toks * a.k_token + dof,
           (kPow2 ? lane_v : vg) + page * a.v_block + toks * a.v_token + dof);
    }
  };
  // Sub-block j straight into LDS stage `stage` (global_load_lds_dwordx4: lane
  // l's 16 bytes land at M0 + 16 l, the slots described above). The loads
  // are issued as inline assembly so that the compiler neither waits for them
  // nor orders LDS reads behind them; the pipeline waits explicitly
  // (vm_wait below) before the barrier that publishes a stage.
  // Page ids are read for all of this wave's instructions before the first
  // load is issued: the loads are `asm volatile` with a memory clobber, so a
  // page-id read placed after one could not move ahead of it, and each
  // instruction would wait for its own LDS round trip.
  auto dma = [&](int j, auto stage_c) {
    constexpr int stage = decltype(stage_c)::value;
    const uint32_t kl = lds_offset(ks[stage]) + 1024 * wave;
    const uint32_t vl = lds_offset(vs[stage]) + 1024 * wave;
    const int k0 = j * kSB;
    auto skip = [&](int r) { return SB_INST % kWaves != 0 && wave + kWaves * r >= SB_INST; };
    if (kPow2 && a.uniform_pages && a.same_kv32 && lane_off32 && k0 + kSB <= end) {
      {
        const int last_page = page_of(k0 + kSB - 1);
        if (last_page >= tbl_base + kTableSeg) load_table(page_of(k0));
      }
      uint64_t off[NI];
#pragma unroll
      for (int r = 0; r < NI; ++r) {
        const int pb = k0 + IR * (wave + kWaves * r);
        const uint32_t page = __builtin_amdgcn_readfirstlane(
            tbl_lds[skip(r) ? 0 : (pb >> a.bs_shift) - tbl_base]);
        const uint32_t row_off = __builtin_amdgcn_readfirstlane(pb & (a.block_size - 1));
        off[r] = (uint64_t)page * (uint32_t)a.k_block + (uint64_t)row_off * (uint32_t)a.k_token;
      }
#pragma unroll
      for (int r = 0; r < NI; ++r) {
        if (skip(r)) continue;  // no such instruction
        lds_dma16_s(kg + off[r], lane_koff, __builtin_amdgcn_readfirstlane(kl + 1024 * kWaves * r));
        lds_dma16_s(vg + off[r], lane_koff, __builtin_amdgcn_readfirstlane(vl + 1024 * kWaves * r));
      }
      return;
    }
    const T* kp[NI];
    const T* vp[NI];
#pragma unroll
    for (int r = 0; r < NI; ++r) kp[r] = vp[r] = nullptr;
    gather_to(j, [&](int r, const T* k, const T* v) {
      kp[r] = k;
      vp[r] = v;
    });
#pragma unroll
    for (int r = 0; r < NI; ++r) {
      if (skip(r)) continue;
      lds_dma16(kp[r], __builtin_amdgcn_readfirstlane(kl + 1024 * kWaves * r));
      lds_dma16(vp[r], __builtin_amdgcn_readfirstlane(vl + 1024 * kWaves * r));
    }
  };
  // Per-lane LDS byte offsets inside a half-stage (the swizzle depends on
  // row & 15, which the 16-key steps below leave unchanged):
  //  * K operand reads: row `col`, dims 16c + 8half;
  //  * transposed V reads: rows 4half + (lane & 15) / 4 (+ 8), dims 32db + tr_col.
  const int tr_row = 4 * half + ((lane & 15) >> 2);
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  // For 256-byte rows (D = 128) the swizzle gives these offsets in closed
  // form, a per-lane base plus an XOR term of the compile-time index:
  //   K chunk c:   kb0 + ((c ^ kt) << 5),
  //   V block db:  vb[h] + ((db ^ vt) << 6)   (row + 8h flips only swizzle bits 0-1),
  // which keeps 5 VGPRs live instead of 16; other head dims keep a table.
  uint32_t koff[DC], voff[DB][2];
#pragma unroll
  for (int c = 0; c < DC; ++c) koff[c] = 2 * L::at(col, 16 * c + 8 * half);
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int h = 0; h < 2; ++h) voff[db][h] = 2 * L::at(tr_row + 8 * h, 32 * db + tr_col);
  const uint32_t kb0 = col * 256 + ((half ^ (L::swizzle(col) & 1)) << 4);
  const uint32_t kt = L::swizzle(col) >> 1;
  const uint32_t vb0 = tr_row * 256 + (((tr_col >> 3) ^ (L::swizzle(tr_row) & 3)) << 4) + (tr_col & 7) * 2;
  const uint32_t vb1 =
      (tr_row + 8) * 256 + (((tr_col >> 3) ^ (L::swizzle(tr_row + 8) & 3)) << 4) + (tr_col & 7) * 2;
  const uint32_t vt = L::swizzle(tr_row) >> 2;
  auto k_offset = [&](int c) -> uint32_t {
    if constexpr (KCH == 16) return kb0 + ((c ^ kt) << 5);
    else return koff[c];
  };
  auto v_offset = [&](int db, int h) -> uint32_t {
    if constexpr (KCH == 16) return (h ? vb1 : vb0) + ((db ^ vt) << 6);
    else return voff[db][h];
  };

  // P^T B-operands of scores `st` (already masked, m current): per 16-key
  // chunk c, elements 8c .. 8c+7 of st, i.e. keys 16c + 4half + {0..3} and
  // 16c + 8 + 4half + {0..3}.
  auto probs = [&](const f32x16& st, u32x4 (&pop)[2]) {
    float p[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] = fast_exp2(fmaf(st[i], a.scale_log2, -m));
#pragma unroll
    for (int c = 0; c < 2; ++c)
      pop[c] = u32x4{pack2<T>(p[8 * c], p[8 * c + 1]), pack2<T>(p[8 * c + 2], p[8 * c + 3]),
                     pack2<T>(p[8 * c + 4], p[8 * c + 5]), pack2<T>(p[8 * c + 6], p[8 * c + 7])};
    // Pairwise sum: a dependency chain of 4 adds instead of 16.
#pragma unroll
    for (int w = 1; w < 16; w *= 2)
#pragma unroll
      for (int i = 0; i < 16; i += 2 * w) p[i] += p[i + w];
    lsum += p[0];
  };
  // Causal / end mask of sub-block j (only where needed: the wave-uniform
  // test passes for sub-blocks entirely below this wave's first query and
  // before `end`), the running max over the lane pair (l, l ^ 32), and the
  // lazy rescale: the reference max (log2 domain, finite from the start)
  // only moves when some lane's max grows by more than 8, so P stays <= 2^8
  // and most sub-blocks skip the O rescale.
  auto unmasked = [&](int j) {
    const int k0 = j * kSB;
    return k0 + kSB <= end && k0 + kSB - 1 <= wave_qpos0;
  };
  // This lane's max over sub-block j's scores; with masked_c true the causal
  // / end mask is first applied to st in place.
  auto row_max = [&](int j, f32x16& st, auto masked_c) {
    const int k0 = j * kSB;
    float mx = -INFINITY;
    if constexpr (!decltype(masked_c)::value) {
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, st[e]);
    } else {
      // Key k0 + 4half + o (o = 8(e / 4) + e % 4) is visible when it is at
      // most lim = min(qpos, end - 1) (-1 for a padding query): one compare
      // against a per-lane bound per score.
      const int bound = (q_ok ? min(qpos, end - 1) : -1) - k0 - 4 * half;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        st[e] = 8 * (e >> 2) + (e & 3) <= bound ? st[e] : -INFINITY;
        mx = fmaxf(mx, st[e]);
      }
    }
    return mx;
  };
  // Max over the lane pair and the lazy rescale of O and the partial sum.
  auto rescale = [&](float mx) {
    {
      // Max with lane l ^ 32: one v_permlane32_swap gives both halves.
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx),
                                                       false, false);
      mx = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    const float mcand = mx * a.scale_log2;
    if (__any(mcand > m + 8.f)) {
      const float mnew = fmaxf(m, mcand);
      const float corr = fast_exp2(m - mnew);
      lsum *= corr;
#pragma unroll
      for (int t2 = 0; t2 < DB; ++t2) acc[t2] *= corr;
      m = mnew;
    }
  };
  auto mask_max = [&](int j, f32x16& st) {
    if (unmasked(j)) rescale(row_max(j, st, std::false_type{}));
    else rescale(row_max(j, st, std::true_type{}));
  };

  // Pipeline over 32-key sub-blocks, three LDS stages, sub-block j in stage
  // j % 3. Step j:
  //   wait until sub-block j has landed (only the loads of j + 1, issued one
  //   step ago, may still be in flight); barrier (sub-block j is visible to
  //   every wave; every wave has finished step j - 1, the last reader of the
  //   stage of j - 1);
  //   load sub-block j + 2 straight into that stage (two steps of latency);
  //   S^T = K Q^T of sub-block j, its mask, row max and lazy rescale, the
  //   probabilities, then O^T += V^T P^T. Each K and V^T operand is read from
  //   LDS one MFMA ahead of its use (two operands live at most), which keeps
  //   the wave within the register budget of three waves per SIMD.
  // The loop is unrolled by kStages so every stage address is a
  // compile-time offset.
  using H0 = std::integral_constant<int, 0>;
  using H1 = std::integral_constant<int, 1>;
  using H2 = std::integral_constant<int, 2>;
  constexpr int kDmaPerStep = 2 * NI;  // K and V loads per wave per sub-block
  // Where the staging loads do not divide evenly (head dims 32 and 96), the
  // first SB_INST % kWaves waves issue NI loads of K and of V per sub-block
  // and the others NI - 1: each wave bounds vmcnt by its own count.
  const bool full_share = SB_INST % kWaves == 0 || wave < SB_INST % kWaves;
  auto dma_wait_newest = [&]() {  // every sub-block but the newest has landed
    if (full_share) vm_wait<kDmaPerStep>();
    else vm_wait<2 * (NI - 1)>();
  };
  if (nsub > 0) {
    dma(0, H0{});
    if (nsub > 1) dma(1, H1{});
    auto step = [&](int j, auto hc) {
      constexpr int h = decltype(hc)::value;
      using Hd = std::integral_constant<int, (h + 2) % kStages>;
      if (j + 1 < nsub) dma_wait_newest();
      else vm_wait<0>();
      __syncthreads();
      if (j + 2 < nsub) dma(j + 2, Hd{});
      if (j >= nsub_w) return;
      const char* kd = reinterpret_cast<const char*>(ks[h]);
      f32x16 st = f32x16{};
      // Each operand is read one MFMA ahead of its use, so a read's latency
      // overlaps the MFMA before it (two in flight per wave at most, which
      // the register budget of three waves per SIMD allows).
      auto kread = [&](int c) { return *reinterpret_cast<const u32x4*>(kd + k_offset(c)); };
      u32x4 kop[DC];
      kop[0] = kread(0);
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        if (c + 1 < DC) kop[c + 1] = kread(c + 1);
        st = Mfma<T>::run(kop[c], qop[c], st);
      }
      mask_max(j, st);
      u32x4 pop[2];
      probs(st, pop);
      // V^T A-operands: lane l needs dim 32db + l % 32 at keys 16c + 4half +
      // {0..3} and 16c + 8 + 4half + {0..3} (pop's k-slots): two transposed
      // reads whose 16-lane group g covers dims 32db + 16(g & 1) .. +15
      // (lanes 4i + s address key i, dims +4s).
      // MFMA i takes c = i / DB, db = i % DB: consecutive MFMAs accumulate
      // into different d blocks (each block still adds c = 0 before c = 1).
      const char* vd = reinterpret_cast<const char*>(vs[h]);
      auto vread = [&](int i) {
        const int c = i / DB, db = i % DB;
        const char* vp = vd + 16 * c * D * 2;
        const u32x2 lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(vp + v_offset(db, 0)));
        const u32x2 hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(vp + v_offset(db, 1)));
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
      u32x4 vop[2 * DB];
      vop[0] = vread(0);
#pragma unroll
      for (int i = 0; i < 2 * DB; ++i) {
        if (i + 1 < 2 * DB) vop[i + 1] = vread(i + 1);
        acc[i % DB] = Mfma<T>::run(vop[i], pop[i / DB], acc[i % DB]);
      }
    };
    for (int j = 0; j < nsub; j += kStages) {
      step(j, H0{});
      if (j + 1 >= nsub) break;
      step(j + 1, H1{});
      if (j + 2 >= nsub) break;
      step(j + 2, H2{});
    }
  }
  lsum += shfl_xor_f32(lsum, 32);
  if (!q_ok) return;
  const float inv = fast_rcp(fmaxf(lsum, 1e-30f));
  T* op = reinterpret_cast<T*>(a.out) + (int64_t)(q_begin + qi) * a.o_token + head * a.o_head;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {  // rows 32db + 8gi + 4half + {0..3}
      const int d = 32 * db + 8 * gi + 4 * half;
      *reinterpret_cast<u32x2*>(op + d) =
          u32x2{pack2<T>(acc[db][4 * gi] * inv, acc[db][4 * gi + 1] * inv),
                pack2<T>(acc[db][4 * gi + 2] * inv, acc[db][4 * gi + 3] * inv)};
    }
  }
}

// Longest-first dispatch order of the sequences (list scheduling: a work item
// of n keys costs ~n / 64 tiles, and the hardware starts workgroups in id
// order as slots free up, so the long items must not come last). Rank sort
// in one workgroup: rank(i) = #{j : key_j > key_i or (key_j == key_i and
// j < i)}, so equal keys keep their order and the permutation is stable.
// key = clamped length, or -1 for sequences the MFMA kernel skips.
constexpr int kOrderMax = 2048;  // larger batches keep the identity order
__global__ __launch_bounds__(1024) void prefill_order_kernel(const int32_t* cu, const int32_t* lengths,
                                                             int32_t num_seqs, int32_t skip_q,
                                                             int64_t cap, int32_t* order) {
  __shared__ int32_t key[kOrderMax];
  for (int i = threadIdx.x; i < num_seqs; i += blockDim.x) {
    const int q_len = cu[i + 1] - cu[i];
    const int64_t n = lengths[i];
    key[i] = q_len <= skip_q ? -1 : (int32_t)(n < 0 ? 0 : (n > cap ? cap : n));
  }
  __syncthreads();
  for (int i = threadIdx.x; i < num_seqs; i += blockDim.x) {
    const int32_t ki = key[i];
    int rank = 0;
    for (int j = 0; j < num_seqs; ++j) {
      const int32_t kj = key[j];
      rank += (kj > ki) | ((kj == ki) & (j < i));
    }
    order[rank] = i;
  }
}

template <typename T, int MODE>
bool launch_prefill_d(int d, dim3 grid, hipStream_t s, const PrefillArgs& a) {
  switch (d) {
#define VRH_D(DV)                                                                          \
  case DV:                                                                                 \
    hipLaunchKernelGGL((paged_prefill_kernel<T, DV, MODE>), grid, dim3(kThreads), 0, s, a); \
    return true;
    VRH_D(32)
    VRH_D(64)
    VRH_D(96)
    VRH_D(128)
#undef VRH_D
    default: return false;
  }
}

template <typename T>
bool launch_prefill(int d, dim3 grid, hipStream_t s, const PrefillArgs& a) {
  if (a.bs_shift >= 0) return launch_prefill_d<T, kShift>(d, grid, s, a);
  return launch_prefill_d<T, kDiv>(d, grid, s, a);
}

}  // namespace
}  // namespace vrh

using namespace vrh;

// Sequences with at most this many queries (decode rows riding in a packed
// batch) run through the split-KV decode kernel instead of MFMA tiles.
constexpr int kDecodeQ = 1;
// A batch whose sequences all have at most kExactQ queries (max_seqlen_q <=
// kExactQ: speculative verification, decode-only batches) runs every query as
// a decode row, so each packed query reproduces single-query decode bit for
// bit (the decode partition depends only on the row's own length).
constexpr int kExactQ = 8;

// Queries per sequence that the decode kernel handles (rows per sequence of
// its expanded grid).
static int decode_route_q(int32_t max_seqlen_q) {
  return max_seqlen_q >= 1 && max_seqlen_q <= kExactQ ? max_seqlen_q : kDecodeQ;
}

// Workspace: split-KV partials of the decode rows, then the dispatch order
// (int32 per sequence, 256-byte aligned).
static size_t decode_part_bytes(int64_t num_seqs, int32_t max_seqlen_q, int32_t q_heads,
                                int32_t head_dim) {
  const int64_t rows = num_seqs * decode_route_q(max_seqlen_q);
  return (vrh_paged_decode_workspace_bytes(rows, q_heads, head_dim) + 255) / 256 * 256;
}

extern "C" size_t vrh_paged_prefill_workspace_bytes(int64_t num_seqs, int32_t max_seqlen_q,
                                                    int32_t q_heads, int32_t head_dim) {
  return decode_part_bytes(num_seqs, max_seqlen_q, q_heads, head_dim) +
         (size_t)num_seqs * sizeof(int32_t);
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
  VRH_CHECK_ARG(num_seqs < (1ll << 31) / kExactQ, "vrh_paged_prefill: too many sequences");
  if (num_seqs == 0 || total_q == 0) return VRH_OK;
  VRH_CHECK_ARG(out && q && key_cache && value_cache && block_tables && context_lengths &&
                    cu_seqlens_q,
                "vrh_paged_prefill: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const bool half = dtype == VRH_DTYPE_BF16 || dtype == VRH_DTYPE_F16;
  bool mfma = half && head_dim % 32 == 0 && head_dim <= 128 && block_size >= 1 &&
              q_token_stride % 8 == 0 && q_head_stride % 8 == 0 && out_token_stride % 4 == 0 &&
              out_head_stride % 4 == 0 && k_block_stride % 8 == 0 && k_token_stride % 8 == 0 &&
              k_head_stride % 8 == 0 && v_block_stride % 8 == 0 && v_token_stride % 8 == 0 &&
              v_head_stride % 8 == 0;
  for (const void* p : {(const void*)out, q, key_cache, value_cache}) mfma = mfma && ((uintptr_t)p % 16 == 0);
  const bool route_decode =
      workspace != nullptr &&
      workspace_bytes >= vrh_paged_prefill_workspace_bytes(num_seqs, max_seqlen_q, q_heads, head_dim);
  const int route_q = decode_route_q(max_seqlen_q);
  if (!mfma) {
    // Every query is a decode row: with a workspace and max_seqlen_q <=
    // kExactQ through the split-KV rows that single-query decode uses (bit
    // for bit the same), otherwise one split per row.
    const bool exact = route_decode && route_q == max_seqlen_q;
    return vrh_decode_rows(dtype, out, q, key_cache, value_cache, block_tables, context_lengths,
                           cu_seqlens_q, (int32_t)num_seqs, exact ? route_q : 0,
                           exact ? num_seqs * route_q : total_q, q_heads, kv_heads, head_dim,
                           block_size, table_width, table_stride, q_token_stride, q_head_stride,
                           out_token_stride, out_head_stride, k_block_stride, k_token_stride,
                           k_head_stride, v_block_stride, v_token_stride, v_head_stride, 0,
                           exact ? workspace : nullptr,
                           exact ? decode_part_bytes(num_seqs, max_seqlen_q, q_heads, head_dim) : 0,
                           s, "vrh_paged_prefill");
  }
  VRH_CHECK_ARG(max_seqlen_q >= 1, "vrh_paged_prefill: max_seqlen_q must be positive");
  VRH_CHECK_ARG(q_heads <= 65535, "vrh_paged_prefill: too many heads");
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
  a.skip_q = route_decode ? route_q : 0;
  {
    // Rows one staging instruction covers: 64 lanes of 16 bytes over rows of
    // head_dim / 8 chunks; the fast addressing needs them on one page.
    const int chunks = head_dim / 8;
    const bool pow2_chunks = (chunks & (chunks - 1)) == 0;
    a.uniform_pages = pow2_chunks && a.bs_shift >= 0 && block_size % (64 / chunks) == 0;
  }
  a.same_kv32 = k_block_stride == v_block_stride &&
                k_token_stride == v_token_stride && k_block_stride >= 0 &&
                k_block_stride < (1ll << 31) && k_token_stride >= 0 &&
                k_token_stride < (1ll << 31);
  a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)head_dim));
  a.num_seqs = num_seqs;
  a.kv_heads = kv_heads;
  a.qblocks = ceil_div(max_seqlen_q, kBM);
  a.order = nullptr;
  // Up to 64 sequences are ranked inside the kernel (also without a
  // workspace); larger batches use the ordering kernel and the workspace.
  a.rank_in_kernel = num_seqs > 1 && num_seqs <= 64;
  // With every sequence routed to the decode kernel (max_seqlen_q <= the
  // routed query count) the MFMA launch, and its ordering, would have no work.
  const bool mfma_work = a.skip_q < max_seqlen_q;
  if (mfma_work && route_decode && num_seqs > 1 && num_seqs <= kOrderMax && !a.rank_in_kernel) {
    int32_t* order = reinterpret_cast<int32_t*>(
        static_cast<char*>(workspace) + decode_part_bytes(num_seqs, max_seqlen_q, q_heads, head_dim));
    hipLaunchKernelGGL(prefill_order_kernel, dim3(1), dim3(1024), 0, s, cu_seqlens_q,
                       context_lengths, (int32_t)num_seqs, a.skip_q,
                       (int64_t)table_width * block_size, order);
    a.order = order;
  }
  const int64_t groups = num_seqs * kv_heads;
  const int64_t launched = (groups + 7) / 8 * 8 * (int64_t)a.group * a.qblocks;
  VRH_CHECK_ARG(launched < (1ll << 31), "vrh_paged_prefill: too many work items");
  if (mfma_work) {
    const bool ok = dtype == VRH_DTYPE_BF16
                        ? launch_prefill<bf16_t>(head_dim, dim3((unsigned)launched), s, a)
                        : launch_prefill<f16_t>(head_dim, dim3((unsigned)launched), s, a);
    VRH_CHECK_ARG(ok, "vrh_paged_prefill: no kernel for head_dim %d", head_dim);
  }
  if (route_decode) {
    // Short sequences of the packed batch: one split-KV decode row per query
    // (row r is query r % route_q of sequence r / route_q).
    const int rc = vrh_decode_rows(
        dtype, out, q, key_cache, value_cache, block_tables, context_lengths, cu_seqlens_q,
        (int32_t)num_seqs, route_q, num_seqs * route_q, q_heads, kv_heads, head_dim,
        block_size, table_width, table_stride, q_token_stride, q_head_stride, out_token_stride,
        out_head_stride, k_block_stride, k_token_stride, k_head_stride, v_block_stride,
        v_token_stride, v_head_stride, 0, workspace,
        decode_part_bytes(num_seqs, max_seqlen_q, q_heads, head_dim), s, "vrh_paged_prefill");
    if (rc != VRH_OK) return rc;
  }
  VRH_RETURN_LAUNCH("vrh_paged_prefill");
}
