// KV append: scatter one [kv_heads, head_dim] token slot per row into the
// paged pool, for one layer view or a batch of layers in one launch.
//
// Reference behaviour: kv_cache_manager.py:689-699 (index_put),
// kernels/routing.py:180-205 (masked store), kernels/graph_kv.py:7-46
// (active_rows + write_mask, int64 address math).
//
// The copy is dtype-free: each thread moves one VECB-byte vector of K and the
// matching vector of V. A job is one (layer, row); a workgroup covers 256
// vectors of one job, so the 4 KiB bf16 K slot of an Ouro token (16 heads x 128)
// is exactly one 256-thread workgroup of 16-byte vectors. Loads of k/v are
// ordinary (they were just written by the projection); stores are the only HBM
// writes of the path, go out as full 64-byte-aligned lines and are
// non-temporal: each slot is written once, and its next reader (the attention
// of the step) reads whole contexts from HBM.
#include "common.h"

namespace vrh {
namespace {

struct AppendArgs {
  char* kc;
  char* vc;
  const char* k;
  const char* v;
  const int64_t* blocks;
  const int64_t* offsets;
  const uint8_t* mask;
  const int32_t* active;
  // byte strides
  int64_t c_block, c_token, c_head, c_layer;
  int64_t k_row, k_head, k_layer;
  int64_t v_row, v_head, v_layer;
  int64_t row_base;
  int64_t num_blocks;     // > 0: rows whose block id is outside [0, num_blocks) are skipped
  int32_t block_size;     // > 0: rows whose offset is outside [0, block_size) are skipped
  int32_t vecs_per_head;  // head bytes / VECB
  int32_t vec_shift;      // log2(vecs_per_head) or -1
  int32_t vecs_per_row;   // kv_heads * vecs_per_head
};

template <int VECB>
__global__ __launch_bounds__(256) void kv_append_kernel(AppendArgs a) {
  using raw_t = raw_of<VECB>;
  const int64_t row = a.row_base + blockIdx.y;  // one job per (row, layer)
  if (a.active != nullptr && row >= (int64_t)(*a.active)) return;
  if (a.mask != nullptr && a.mask[row] == 0) return;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= a.vecs_per_row) return;
  int h, jj;
  if (a.vec_shift >= 0) {
    h = j >> a.vec_shift;
    jj = j & (a.vecs_per_head - 1);
  } else {
    h = j / a.vecs_per_head;
    jj = j - h * a.vecs_per_head;
  }
  const int64_t lay = blockIdx.z;
  const int64_t block = a.blocks[row], offset = a.offsets[row];
  // Out-of-range addresses write nothing (the pool is never written outside
  // its blocks); in range is the caller's contract, as in the reference.
  if (a.num_blocks > 0 && (block < 0 || block >= a.num_blocks)) return;
  if (a.block_size > 0 && (offset < 0 || offset >= a.block_size)) return;
  // Block ids are promoted to 64 bits before the multiply: pools exceed 2^31 B.
  const int64_t dst = block * a.c_block + offset * a.c_token + h * a.c_head +
                      lay * a.c_layer + (int64_t)jj * VECB;
  const raw_t kv = *reinterpret_cast<const raw_t*>(a.k + row * a.k_row + h * a.k_head +
                                                   lay * a.k_layer + (int64_t)jj * VECB);
  const raw_t vv = *reinterpret_cast<const raw_t*>(a.v + row * a.v_row + h * a.v_head +
                                                   lay * a.v_layer + (int64_t)jj * VECB);
  __builtin_nontemporal_store(kv, reinterpret_cast<raw_t*>(a.kc + dst));
  __builtin_nontemporal_store(vv, reinterpret_cast<raw_t*>(a.vc + dst));
}

}  // namespace
}  // namespace vrh

using namespace vrh;

extern "C" int vrh_kv_append(int dtype, void* key_cache, void* value_cache,
                             int64_t cache_block_stride, int64_t cache_token_stride,
                             int64_t cache_head_stride, int64_t cache_layer_stride,
                             const void* k, const void* v, int64_t k_row_stride,
                             int64_t k_head_stride, int64_t k_layer_stride,
                             int64_t v_row_stride, int64_t v_head_stride,
                             int64_t v_layer_stride, const int64_t* write_blocks,
                             const int64_t* write_offsets, const uint8_t* write_mask,
                             const int32_t* active_rows, int64_t rows, int32_t layers,
                             int32_t kv_heads, int32_t head_dim, int64_t num_blocks,
                             int32_t block_size, vrh_stream_t stream) {
  const int es = dtype_bytes(dtype);
  VRH_CHECK_ARG(es > 0, "vrh_kv_append: unknown dtype %d", dtype);
  VRH_CHECK_ARG(rows >= 0 && layers >= 1 && kv_heads >= 1 && head_dim >= 1,
                "vrh_kv_append: bad sizes rows=%lld layers=%d kv_heads=%d head_dim=%d",
                (long long)rows, layers, kv_heads, head_dim);
  VRH_CHECK_ARG(layers <= 65535, "vrh_kv_append: at most 65535 layers per launch");
  if (rows == 0) return VRH_OK;
  VRH_CHECK_ARG(key_cache && value_cache && k && v && write_blocks && write_offsets,
                "vrh_kv_append: null pointer");
  AppendArgs a;
  a.kc = (char*)key_cache;
  a.vc = (char*)value_cache;
  a.k = (const char*)k;
  a.v = (const char*)v;
  a.blocks = write_blocks;
  a.offsets = write_offsets;
  a.mask = write_mask;
  a.active = active_rows;
  a.c_block = cache_block_stride * es;
  a.c_token = cache_token_stride * es;
  a.c_head = cache_head_stride * es;
  a.c_layer = cache_layer_stride * es;
  a.k_row = k_row_stride * es;
  a.k_head = k_head_stride * es;
  a.k_layer = k_layer_stride * es;
  a.v_row = v_row_stride * es;
  a.v_head = v_head_stride * es;
  a.v_layer = v_layer_stride * es;
  a.row_base = 0;
  a.num_blocks = num_blocks;
  a.block_size = block_size;
  const int64_t head_bytes = (int64_t)head_dim * es;
  const int vb = pick_vb({head_bytes, a.c_block, a.c_token, a.c_head, a.c_layer, a.k_row,
                          a.k_head, a.k_layer, a.v_row, a.v_head, a.v_layer},
                         {key_cache, value_cache, k, v});
  a.vecs_per_head = (int32_t)(head_bytes / vb);
  a.vec_shift = -1;
  if ((a.vecs_per_head & (a.vecs_per_head - 1)) == 0) {
    a.vec_shift = __builtin_ctz((unsigned)a.vecs_per_head);
  }
  const int64_t vpr = (int64_t)kv_heads * a.vecs_per_head;
  VRH_CHECK_ARG(vpr < (1ll << 30), "vrh_kv_append: token slot too large");
  a.vecs_per_row = (int32_t)vpr;
  // Rows go on grid.y (<= 65535 per launch); layers on grid.z.
  hipStream_t s = (hipStream_t)stream;
  const unsigned gx = (unsigned)ceil_div64(vpr, 256);
  for (int64_t first = 0; first < rows; first += 65535) {
    AppendArgs part = a;
    const int64_t count = rows - first < 65535 ? rows - first : 65535;
    part.row_base = first;
    dim3 grid(gx, (unsigned)count, (unsigned)layers);
    VRH_DISPATCH_VB(vb, kv_append_kernel, grid, dim3(256), s, part)
  }
  VRH_RETURN_LAUNCH("vrh_kv_append");
}
