// Bit-exact KV movement kernels: whole-block copy (preemption snapshot/restore
// staging and copy-on-write), LAST_EXITED depth propagation (finalize) and the
// block-table gather that materialises a request's history (read).
//
// All of them are byte copies, so they are written once over raw bytes with the
// widest vector (16, 8, 4, 2 or 1 bytes) that every pointer and stride allows.
//
// Reference behaviour:
//   copy_blocks    on-device block copy (copy-on-write / compaction)
//   blocks_to_host / blocks_from_host
//                  kv_cache_manager.py:481-523 (snapshot/restore: the page
//                  copies to and from host memory, batched into one launch)
//   finalize       kernels/routing.py:147-177 (finalize_kernel), launched as in
//                  worker/model_runner.py:1331-1346
//   finalize_token kv_cache_manager.py:806-831
//   gather         kv_cache_manager.py:834-854 (read)
#include <algorithm>

#include "common.h"


namespace vrh {
namespace {

// ------------------------------------------------------------ block copy
// grid.x tiles one block (kUnroll * 256 vectors per workgroup), grid.y = pair.
constexpr int kCopyUnroll = 4;

struct CopyBlocksArgs {
  char* kc;
  char* vc;
  const int64_t* src;
  const int64_t* dst;
  int64_t block_stride;  // bytes
  int64_t vecs;          // vectors per block
  int64_t pair_base;
};

template <int VB>
__global__ __launch_bounds__(256) void copy_blocks_kernel(CopyBlocksArgs a) {
  using raw_t = raw_of<VB>;
  const int64_t pair = a.pair_base + blockIdx.y;
  const int64_t s = a.src[pair] * a.block_stride;
  const int64_t d = a.dst[pair] * a.block_stride;
  const int64_t first = (int64_t)blockIdx.x * (256 * kCopyUnroll) + threadIdx.x;
  raw_t kr[kCopyUnroll], vr[kCopyUnroll];
#pragma unroll
  for (int u = 0; u < kCopyUnroll; ++u) {
    const int64_t i = first + u * 256;
    if (i < a.vecs) {
      kr[u] = __builtin_nontemporal_load(reinterpret_cast<const raw_t*>(a.kc + s) + i);
      vr[u] = __builtin_nontemporal_load(reinterpret_cast<const raw_t*>(a.vc + s) + i);
    }
  }
#pragma unroll
  for (int u = 0; u < kCopyUnroll; ++u) {
    const int64_t i = first + u * 256;
    if (i < a.vecs) {
      __builtin_nontemporal_store(kr[u], reinterpret_cast<raw_t*>(a.kc + d) + i);
      __builtin_nontemporal_store(vr[u], reinterpret_cast<raw_t*>(a.vc + d) + i);
    }
  }
}

// ---------------------------------------------------- slot (token) copies
// A "slot" is the channel_bytes of one (block, layer, token). Jobs enumerate
// (row, target plane, layer); each thread moves one vector of K and of V.
struct FinalizeArgs {
  char* kc;
  char* vc;
  const int64_t* desc;
  const int32_t* tables;
  int64_t row_base;
  int32_t planes, width, page, layers;
  int64_t block_stride, layer_stride, token_stride;  // bytes
  int32_t vecs;                                      // vectors per slot
};

template <int VB>
__global__ __launch_bounds__(256) void finalize_kernel(FinalizeArgs a) {
  using raw_t = raw_of<VB>;
  const int64_t row = a.row_base + blockIdx.y;
  const int target = blockIdx.z % a.planes;
  const int layer = blockIdx.z / a.planes;
  const int64_t slot = a.desc[row * 3 + 0];
  const int64_t depth = a.desc[row * 3 + 1];
  const int64_t pos = a.desc[row * 3 + 2];
  if (target <= depth) return;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= a.vecs) return;
  const int64_t page = pos / a.page;
  const int64_t src = a.tables[(slot * a.planes + depth) * a.width + page];
  const int64_t dst = a.tables[(slot * a.planes + target) * a.width + page];
  const int64_t off = (int64_t)layer * a.layer_stride + (pos % a.page) * a.token_stride;
  const raw_t* ks = reinterpret_cast<const raw_t*>(a.kc + src * a.block_stride + off);
  const raw_t* vs = reinterpret_cast<const raw_t*>(a.vc + src * a.block_stride + off);
  raw_t* kd = reinterpret_cast<raw_t*>(a.kc + dst * a.block_stride + off);
  raw_t* vd = reinterpret_cast<raw_t*>(a.vc + dst * a.block_stride + off);
  // Non-temporal stores: the deeper planes' slots are written once here and
  // read by later steps' attention, which streams whole contexts.
  __builtin_nontemporal_store(ks[j], kd + j);
  __builtin_nontemporal_store(vs[j], vd + j);
}

constexpr int kMaxTokenDst = 64;
constexpr int kMaxTokenLayers = 256;

struct FinalizeTokenArgs {
  char* kc;
  char* vc;
  int64_t src;
  int64_t block_stride, layer_stride, token_stride;
  int64_t token_off;  // offset * token_stride
  int32_t vecs;
  int64_t dst[kMaxTokenDst];
  int16_t layers[kMaxTokenLayers];
};

template <int VB>
__global__ __launch_bounds__(256) void finalize_token_kernel(FinalizeTokenArgs a) {
  using raw_t = raw_of<VB>;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= a.vecs) return;
  const int64_t off = (int64_t)a.layers[blockIdx.y] * a.layer_stride + a.token_off;
  const int64_t dst = a.dst[blockIdx.z];
  const raw_t k = reinterpret_cast<const raw_t*>(a.kc + a.src * a.block_stride + off)[j];
  const raw_t v = reinterpret_cast<const raw_t*>(a.vc + a.src * a.block_stride + off)[j];
  reinterpret_cast<raw_t*>(a.kc + dst * a.block_stride + off)[j] = k;
  reinterpret_cast<raw_t*>(a.vc + dst * a.block_stride + off)[j] = v;
}

// ---------------------------------------------------------------- gather
struct GatherArgs {
  char* ok;
  char* ov;
  const char* kc;
  const char* vc;
  const int32_t* table;
  int64_t token_base;
  int32_t page;
  int64_t block_stride, token_stride, channel;  // bytes
  int32_t vecs;
};

template <int VB>
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs a) {
  using raw_t = raw_of<VB>;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= a.vecs) return;
  const int64_t t = a.token_base + blockIdx.y;
  const int64_t blk = a.table[t / a.page];
  const int64_t src = blk * a.block_stride + (t % a.page) * a.token_stride;
  reinterpret_cast<raw_t*>(a.ok + t * a.channel)[j] =
      reinterpret_cast<const raw_t*>(a.kc + src)[j];
  reinterpret_cast<raw_t*>(a.ov + t * a.channel)[j] =
      reinterpret_cast<const raw_t*>(a.vc + src)[j];
}

constexpr int64_t kMaxGridY = 65535;

// ------------------------------------------------- host offload (snapshot)
// Whole blocks between the pool and pinned host rows (row i <-> blocks[i]),
// read or written by the kernel through the host memory's device mapping: one
// launch per direction and no device staging buffer. grid.x tiles a block
// (kCopyUnroll * 256 vectors per workgroup, all loads issued before the
// stores to keep many host-link transfers in flight), grid.y = block.
struct HostCopyArgs {
  char* kc;
  char* vc;
  char* hk;  // device address of the pinned host rows
  char* hv;
  const int64_t* blocks;
  int64_t block_stride;  // bytes between pool blocks
  int64_t block_bytes;   // bytes per block = bytes per host row
  int64_t vecs;
  int64_t base;
};

template <int VB, bool TO_HOST>
__device__ __forceinline__ void host_copy_body(const HostCopyArgs& a) {
  using raw_t = raw_of<VB>;
  const int64_t row = a.base + blockIdx.y;
  const int64_t pool_off = a.blocks[row] * a.block_stride;
  const int64_t host_off = row * a.block_bytes;
  const raw_t* ks = reinterpret_cast<const raw_t*>((TO_HOST ? a.kc + pool_off : a.hk + host_off));
  const raw_t* vs = reinterpret_cast<const raw_t*>((TO_HOST ? a.vc + pool_off : a.hv + host_off));
  raw_t* kd = reinterpret_cast<raw_t*>(TO_HOST ? a.hk + host_off : a.kc + pool_off);
  raw_t* vd = reinterpret_cast<raw_t*>(TO_HOST ? a.hv + host_off : a.vc + pool_off);
  const int64_t first = (int64_t)blockIdx.x * (256 * kCopyUnroll) + threadIdx.x;
  raw_t kr[kCopyUnroll], vr[kCopyUnroll];
#pragma unroll
  for (int u = 0; u < kCopyUnroll; ++u) {
    const int64_t i = first + u * 256;
    if (i < a.vecs) {
      kr[u] = __builtin_nontemporal_load(ks + i);
      vr[u] = __builtin_nontemporal_load(vs + i);
    }
  }
#pragma unroll
  for (int u = 0; u < kCopyUnroll; ++u) {
    const int64_t i = first + u * 256;
    if (i < a.vecs) {
      __builtin_nontemporal_store(kr[u], kd + i);
      __builtin_nontemporal_store(vr[u], vd + i);
    }
  }
}

template <int VB>
__global__ __launch_bounds__(256) void blocks_to_host_kernel(HostCopyArgs a) {
  host_copy_body<VB, true>(a);
}
template <int VB>
__global__ __launch_bounds__(256) void blocks_from_host_kernel(HostCopyArgs a) {
  host_copy_body<VB, false>(a);
}

// Device address of pinned host memory; null if `p` is not host memory that
// the runtime mapped for the device (pageable memory must never reach a
// kernel).
void* host_device_pointer(void* p) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (attr.type != hipMemoryTypeHost) return nullptr;
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, p, 0) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return d;
}

int host_copy(bool to_host, void* key_cache, void* value_cache, int64_t block_stride_bytes,
              int64_t block_bytes, const int64_t* blocks, void* host_keys, void* host_values,
              int64_t n, hipStream_t s, const char* who) {
  VRH_CHECK_ARG(n >= 0 && block_bytes >= 0 && block_stride_bytes >= block_bytes,
                "%s: bad sizes n=%lld block_bytes=%lld stride=%lld", who, (long long)n,
                (long long)block_bytes, (long long)block_stride_bytes);
  if (n == 0 || block_bytes == 0) return VRH_OK;
  VRH_CHECK_ARG(key_cache && value_cache && blocks && host_keys && host_values,
                "%s: null pointer", who);
  HostCopyArgs a;
  a.kc = static_cast<char*>(key_cache);
  a.vc = static_cast<char*>(value_cache);
  a.hk = static_cast<char*>(host_device_pointer(host_keys));
  a.hv = static_cast<char*>(host_device_pointer(host_values));
  VRH_CHECK_ARG(a.hk && a.hv, "%s: host buffers must be pinned host memory (hipHostMalloc)", who);
  a.blocks = blocks;
  a.block_stride = block_stride_bytes;
  a.block_bytes = block_bytes;
  const int vb = pick_vb({block_stride_bytes, block_bytes},
                         {key_cache, value_cache, (const void*)a.hk, (const void*)a.hv});
  a.vecs = block_bytes / vb;
  const int64_t gx = ceil_div64(a.vecs, 256 * kCopyUnroll);
  VRH_CHECK_ARG(gx < (1ll << 31), "%s: block too large", who);
  for (int64_t first = 0; first < n; first += kMaxGridY) {
    a.base = first;
    const dim3 grid((unsigned)gx, (unsigned)std::min(n - first, kMaxGridY));
    if (to_host) VRH_DISPATCH_VB(vb, blocks_to_host_kernel, grid, dim3(256), s, a)
    else VRH_DISPATCH_VB(vb, blocks_from_host_kernel, grid, dim3(256), s, a)
  }
  VRH_RETURN_LAUNCH(who);
}

}  // namespace
}  // namespace vrh

using namespace vrh;

extern "C" int vrh_kv_copy_blocks(void* key_cache, void* value_cache, int64_t block_stride_bytes,
                                  int64_t block_bytes, const int64_t* src_blocks,
                                  const int64_t* dst_blocks, int64_t n, vrh_stream_t stream) {
  VRH_CHECK_ARG(n >= 0 && block_bytes >= 0 && block_stride_bytes >= block_bytes,
                "vrh_kv_copy_blocks: bad sizes n=%lld block_bytes=%lld stride=%lld",
                (long long)n, (long long)block_bytes, (long long)block_stride_bytes);
  if (n == 0 || block_bytes == 0) return VRH_OK;
  VRH_CHECK_ARG(key_cache && value_cache && src_blocks && dst_blocks,
                "vrh_kv_copy_blocks: null pointer");
  const int vb = pick_vb({block_stride_bytes, block_bytes}, {key_cache, value_cache});
  CopyBlocksArgs a;
  a.kc = (char*)key_cache;
  a.vc = (char*)value_cache;
  a.src = src_blocks;
  a.dst = dst_blocks;
  a.block_stride = block_stride_bytes;
  a.vecs = block_bytes / vb;
  const int64_t gx = ceil_div64(a.vecs, 256 * kCopyUnroll);
  VRH_CHECK_ARG(gx < (1ll << 31), "vrh_kv_copy_blocks: block too large");
  hipStream_t s = (hipStream_t)stream;
  for (int64_t first = 0; first < n; first += kMaxGridY) {
    a.pair_base = first;
    const int64_t count = std::min(n - first, kMaxGridY);
    dim3 grid((unsigned)gx, (unsigned)count);
    VRH_DISPATCH_VB(vb, copy_blocks_kernel, grid, dim3(256), s, a);
  }
  VRH_RETURN_LAUNCH("vrh_kv_copy_blocks");
}

extern "C" int vrh_kv_finalize(void* key_cache, void* value_cache, const int64_t* descriptors,
                               const int32_t* tables, int64_t rows, int32_t planes,
                               int32_t width, int32_t block_size, int32_t layers,
                               int64_t block_stride_bytes, int64_t layer_stride_bytes,
                               int64_t token_stride_bytes, int64_t channel_bytes,
                               vrh_stream_t stream) {
  VRH_CHECK_ARG(rows >= 0 && planes >= 1 && width >= 1 && block_size >= 1 && layers >= 1 &&
                    channel_bytes >= 1,
                "vrh_kv_finalize: bad sizes");
  VRH_CHECK_ARG((int64_t)planes * layers <= 65535, "vrh_kv_finalize: planes * layers > 65535");
  if (rows == 0 || planes == 1) return VRH_OK;
  VRH_CHECK_ARG(key_cache && value_cache && descriptors && tables, "vrh_kv_finalize: null pointer");
  const int vb = pick_vb({block_stride_bytes, layer_stride_bytes, token_stride_bytes, channel_bytes},
                         {key_cache, value_cache});
  FinalizeArgs a;
  a.kc = (char*)key_cache;
  a.vc = (char*)value_cache;
  a.desc = descriptors;
  a.tables = tables;
  a.planes = planes;
  a.width = width;
  a.page = block_size;
  a.layers = layers;
  a.block_stride = block_stride_bytes;
  a.layer_stride = layer_stride_bytes;
  a.token_stride = token_stride_bytes;
  VRH_CHECK_ARG(channel_bytes / vb < (1ll << 30), "vrh_kv_finalize: slot too large");
  a.vecs = (int32_t)(channel_bytes / vb);
  hipStream_t s = (hipStream_t)stream;
  for (int64_t first = 0; first < rows; first += kMaxGridY) {
    a.row_base = first;
    const int64_t count = std::min(rows - first, kMaxGridY);
    dim3 grid((unsigned)ceil_div64(a.vecs, 256), (unsigned)count, (unsigned)(planes * layers));
    VRH_DISPATCH_VB(vb, finalize_kernel, grid, dim3(256), s, a);
  }
  VRH_RETURN_LAUNCH("vrh_kv_finalize");
}

extern "C" int vrh_kv_finalize_token(void* key_cache, void* value_cache, int64_t src_block,
                                     const int64_t* dst_blocks, int32_t num_dst, int32_t offset,
                                     const int32_t* layer_ids, int32_t num_layers,
                                     int64_t block_stride_bytes, int64_t layer_stride_bytes,
                                     int64_t token_stride_bytes, int64_t channel_bytes,
                                     vrh_stream_t stream) {
  VRH_CHECK_ARG(num_dst >= 0 && num_dst <= kMaxTokenDst,
                "vrh_kv_finalize_token: num_dst must be in [0, %d]", kMaxTokenDst);
  VRH_CHECK_ARG(num_layers >= 0 && num_layers <= kMaxTokenLayers,
                "vrh_kv_finalize_token: num_layers must be in [0, %d]", kMaxTokenLayers);
  VRH_CHECK_ARG(channel_bytes >= 1 && offset >= 0 && src_block >= 0,
                "vrh_kv_finalize_token: bad sizes");
  if (num_dst == 0 || num_layers == 0) return VRH_OK;
  VRH_CHECK_ARG(key_cache && value_cache && dst_blocks && layer_ids,
                "vrh_kv_finalize_token: null pointer");
  const int vb = pick_vb({block_stride_bytes, layer_stride_bytes, token_stride_bytes, channel_bytes},
                         {key_cache, value_cache});
  FinalizeTokenArgs a;
  a.kc = (char*)key_cache;
  a.vc = (char*)value_cache;
  a.src = src_block;
  a.block_stride = block_stride_bytes;
  a.layer_stride = layer_stride_bytes;
  a.token_stride = token_stride_bytes;
  a.token_off = (int64_t)offset * token_stride_bytes;
  VRH_CHECK_ARG(channel_bytes / vb < (1ll << 30), "vrh_kv_finalize_token: slot too large");
  a.vecs = (int32_t)(channel_bytes / vb);
  for (int i = 0; i < num_dst; ++i) {
    VRH_CHECK_ARG(dst_blocks[i] >= 0 && dst_blocks[i] != src_block,
                  "vrh_kv_finalize_token: destination %d is invalid", i);
    a.dst[i] = dst_blocks[i];
  }
  for (int i = 0; i < num_layers; ++i) {
    VRH_CHECK_ARG(layer_ids[i] >= 0 && layer_ids[i] < 32768,
                  "vrh_kv_finalize_token: layer id %d out of range", layer_ids[i]);
    a.layers[i] = (int16_t)layer_ids[i];
  }
  dim3 grid((unsigned)ceil_div64(a.vecs, 256), (unsigned)num_layers, (unsigned)num_dst);
  VRH_DISPATCH_VB(vb, finalize_token_kernel, grid, dim3(256), (hipStream_t)stream, a);
  VRH_RETURN_LAUNCH("vrh_kv_finalize_token");
}

extern "C" int vrh_kv_gather(void* out_k, void* out_v, const void* key_cache,
                             const void* value_cache, const int32_t* table, int64_t length,
                             int32_t block_size, int64_t block_stride_bytes,
                             int64_t token_stride_bytes, int64_t channel_bytes,
                             vrh_stream_t stream) {
  VRH_CHECK_ARG(length >= 0 && block_size >= 1 && channel_bytes >= 1,
                "vrh_kv_gather: bad sizes");
  if (length == 0) return VRH_OK;
  VRH_CHECK_ARG(out_k && out_v && key_cache && value_cache && table,
                "vrh_kv_gather: null pointer");
  const int vb = pick_vb({block_stride_bytes, token_stride_bytes, channel_bytes},
                         {out_k, out_v, key_cache, value_cache});
  GatherArgs a;
  a.ok = (char*)out_k;
  a.ov = (char*)out_v;
  a.kc = (const char*)key_cache;
  a.vc = (const char*)value_cache;
  a.table = table;
  a.page = block_size;
  a.block_stride = block_stride_bytes;
  a.token_stride = token_stride_bytes;
  a.channel = channel_bytes;
  VRH_CHECK_ARG(channel_bytes / vb < (1ll << 30), "vrh_kv_gather: slot too large");
  a.vecs = (int32_t)(channel_bytes / vb);
  hipStream_t s = (hipStream_t)stream;
  for (int64_t first = 0; first < length; first += kMaxGridY) {
    a.token_base = first;
    const int64_t count = std::min(length - first, kMaxGridY);
    dim3 grid((unsigned)ceil_div64(a.vecs, 256), (unsigned)count);
    VRH_DISPATCH_VB(vb, gather_kernel, grid, dim3(256), s, a);
  }
  VRH_RETURN_LAUNCH("vrh_kv_gather");
}

extern "C" int vrh_kv_blocks_to_host(const void* key_cache, const void* value_cache,
                                     int64_t block_stride_bytes, int64_t block_bytes,
                                     const int64_t* blocks, void* host_keys, void* host_values,
                                     int64_t n, vrh_stream_t stream) {
  return host_copy(true, const_cast<void*>(key_cache), const_cast<void*>(value_cache),
                   block_stride_bytes, block_bytes, blocks, host_keys, host_values, n,
                   (hipStream_t)stream, "vrh_kv_blocks_to_host");
}

extern "C" int vrh_kv_blocks_from_host(void* key_cache, void* value_cache,
                                       int64_t block_stride_bytes, int64_t block_bytes,
                                       const int64_t* blocks, const void* host_keys,
                                       const void* host_values, int64_t n, vrh_stream_t stream) {
  return host_copy(false, key_cache, value_cache, block_stride_bytes, block_bytes, blocks,
                   const_cast<void*>(host_keys), const_cast<void*>(host_values), n,
                   (hipStream_t)stream, "vrh_kv_blocks_from_host");
}
