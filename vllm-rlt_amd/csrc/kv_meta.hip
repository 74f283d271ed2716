// Integer address kernels feeding the append and attention kernels, plus the
// library's error/version plumbing.
//
// Reference behaviour:
//   expand_kv_addresses  kernels/metadata.py:7-24
//   routing_metadata     kernels/routing.py:14-48 (metadata_kernel)
//   routing_slots        kernels/routing.py:7-11 (slots_kernel)
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

static thread_local char g_last_error[512] = "";

void vrh_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

extern "C" const char* vrh_last_error(void) { return g_last_error; }
extern "C" int vrh_abi_version(void) { return 5; }

namespace vrh {
namespace {

__global__ __launch_bounds__(256) void expand_addresses_kernel(
    const int64_t* positions, const int32_t* sequences, const int32_t* tables, int64_t* blocks,
    int64_t* offsets, int64_t n, int32_t width, int32_t page) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t pos = positions[i];
  const int64_t seq = sequences[i];
  blocks[i] = tables[seq * width + pos / page];
  offsets[i] = pos % page;
}

// One workgroup per row: lanes copy the row's table slice while lane 0 writes
// the scalars.
__global__ __launch_bounds__(256) void routing_metadata_kernel(
    const int64_t* desc, const int32_t* tables, int64_t* slots, int64_t* positions,
    int32_t* lengths, int64_t* blocks, int64_t* offsets, int32_t* out_tables, int64_t n,
    int32_t width, int32_t page, int32_t planes, int32_t out_width) {
  const int64_t row = blockIdx.x;
  const bool valid = row < n;
  const int64_t slot = valid ? desc[row * 3 + 0] : 0;
  const int64_t depth = valid ? desc[row * 3 + 1] : 0;
  const int64_t pos = valid ? desc[row * 3 + 2] : 0;
  const int64_t plane = planes > 1 ? depth : 0;
  const int64_t base = (slot * planes + plane) * width;
  if (threadIdx.x == 0) {
    slots[row] = slot;
    positions[row] = pos;
    lengths[row] = valid ? (int32_t)(pos + 1) : 0;
    if (valid) {
      blocks[row] = tables[base + pos / page];
      offsets[row] = pos % page;
    }
  }
  for (int c = threadIdx.x; c < out_width; c += 256) {
    out_tables[row * width + c] = valid ? tables[base + c] : 0;
  }
}

__global__ __launch_bounds__(256) void routing_slots_kernel(const int64_t* desc, int64_t* slots,
                                                            int64_t n, int64_t size) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= size) return;
  slots[r] = r < n ? desc[r * 3] : 0;
}

}  // namespace
}  // namespace vrh

using namespace vrh;

extern "C" int vrh_expand_kv_addresses(const int64_t* positions, const int32_t* sequences,
                                       const int32_t* tables, int64_t* blocks, int64_t* offsets,
                                       int64_t n, int32_t width, int32_t page,
                                       vrh_stream_t stream) {
  VRH_CHECK_ARG(n >= 0 && width >= 0 && page >= 1, "vrh_expand_kv_addresses: bad sizes");
  if (n == 0) return VRH_OK;
  VRH_CHECK_ARG(positions && sequences && tables && blocks && offsets,
                "vrh_expand_kv_addresses: null pointer");
  hipLaunchKernelGGL(expand_addresses_kernel, dim3((unsigned)ceil_div64(n, 256)), dim3(256), 0,
                     (hipStream_t)stream, positions, sequences, tables, blocks, offsets, n, width,
                     page);
  VRH_RETURN_LAUNCH("vrh_expand_kv_addresses");
}

extern "C" int vrh_routing_metadata(const int64_t* descriptors, const int32_t* tables,
                                    int64_t* slots, int64_t* positions, int32_t* lengths,
                                    int64_t* blocks, int64_t* offsets, int32_t* out_tables,
                                    int64_t n, int64_t size, int32_t width, int32_t page,
                                    int32_t planes, int32_t out_width, vrh_stream_t stream) {
  VRH_CHECK_ARG(n >= 0 && size >= n && width >= 1 && page >= 1 && planes >= 1 &&
                    out_width >= 0 && out_width <= width,
                "vrh_routing_metadata: bad sizes n=%lld size=%lld width=%d out_width=%d",
                (long long)n, (long long)size, width, out_width);
  if (size == 0) return VRH_OK;
  VRH_CHECK_ARG(size < (1ll << 31), "vrh_routing_metadata: too many rows");
  VRH_CHECK_ARG(tables && slots && positions && lengths && blocks && offsets && out_tables &&
                    (n == 0 || descriptors),
                "vrh_routing_metadata: null pointer");
  hipLaunchKernelGGL(routing_metadata_kernel, dim3((unsigned)size), dim3(256), 0,
                     (hipStream_t)stream, descriptors, tables, slots, positions, lengths, blocks,
                     offsets, out_tables, n, width, page, planes, out_width);
  VRH_RETURN_LAUNCH("vrh_routing_metadata");
}

extern "C" int vrh_routing_slots(const int64_t* descriptors, int64_t* slots, int64_t n,
                                 int64_t size, vrh_stream_t stream) {
  VRH_CHECK_ARG(n >= 0 && size >= 0, "vrh_routing_slots: bad sizes");
  if (size == 0) return VRH_OK;
  VRH_CHECK_ARG(slots && (n == 0 || descriptors), "vrh_routing_slots: null pointer");
  hipLaunchKernelGGL(routing_slots_kernel, dim3((unsigned)ceil_div64(size, 256)), dim3(256), 0,
                     (hipStream_t)stream, descriptors, slots, n, size);
  VRH_RETURN_LAUNCH("vrh_routing_slots");
}
