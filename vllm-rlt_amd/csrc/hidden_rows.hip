// Hidden-state row movement on either side of packed (WCPB) prefill and of
// async routing: byte copies of whole rows between a slot-indexed pool and a
// batch-ordered buffer.
//
// Reference behaviour (kernels/routing.py:51-144):
//   gather_rows     gather_kernel: out[r] = r < n ? pool[slots[r]] : 0, r < size
//                   (worker/async_state.py:104-113, async_speculative.py:371-380)
//   scatter_rows    scatter_kernel: pool[slots[r]] = in[r], r < count
//                   (worker/async_state.py:115-123)
//   gather_segments gather_segments_kernel: segment s = (slot, offset, count,
//                   start, keep) copies pool rows slot * pool_rows + offset + i
//                   to out rows start + i, i < count
//                   (worker/model_runner.py:515-552)
//   scatter_segments scatter_segments_kernel: the reverse, only when keep != 0
//                   (worker/model_runner.py:554-597)
// Rows are `width` bytes; every pointer and stride is in bytes. The widest
// vector (16..1 bytes) that divides them is used; one thread moves one vector.
#include <algorithm>

#include "common.h"

namespace vrh {
namespace {

constexpr int kThreads = 256;
constexpr int kSegRows = 4;            // rows per workgroup in the segment kernels
constexpr int64_t kMaxGrid = 65535;    // grid.y / grid.z limit

struct RowsArgs {
  const char* src;
  char* dst;
  const int64_t* slots;
  int64_t n;            // gather: rows with a valid slot (the rest are zero-filled)
  int64_t vecs;         // vectors per row
  int64_t src_stride;   // bytes
  int64_t dst_stride;
  int64_t row_base;
};

template <int VB>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(RowsArgs a) {
  using raw_t = raw_of<VB>;
  const int64_t r = a.row_base + blockIdx.y;
  const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (j >= a.vecs) return;
  raw_t v = raw_t{};
  if (r < a.n) v = reinterpret_cast<const raw_t*>(a.src + a.slots[r] * a.src_stride)[j];
  reinterpret_cast<raw_t*>(a.dst + r * a.dst_stride)[j] = v;
}

template <int VB>
__global__ __launch_bounds__(kThreads) void scatter_rows_kernel(RowsArgs a) {
  using raw_t = raw_of<VB>;
  const int64_t r = a.row_base + blockIdx.y;
  const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (j >= a.vecs) return;
  reinterpret_cast<raw_t*>(a.dst + a.slots[r] * a.dst_stride)[j] =
      reinterpret_cast<const raw_t*>(a.src + r * a.src_stride)[j];
}

struct SegmentArgs {
  const char* src;
  char* dst;
  const int64_t* segments;  // [n, 5]: slot, offset, count, batch start, keep
  int64_t pool_rows;
  int64_t vecs;
  int64_t src_stride, dst_stride;
  int64_t seg_base;
};

// GATHER: pool -> batch; otherwise batch -> pool for segments with keep != 0.
template <int VB, bool GATHER>
__device__ __forceinline__ void segments_body(const SegmentArgs& a) {
  using raw_t = raw_of<VB>;
  const int64_t* seg = a.segments + (a.seg_base + blockIdx.z) * 5;
  const int64_t slot = seg[0], offset = seg[1], count = seg[2], start = seg[3];
  if (!GATHER && seg[4] == 0) return;
  const int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (j >= a.vecs) return;
#pragma unroll
  for (int i = 0; i < kSegRows; ++i) {
    const int64_t row = (int64_t)blockIdx.y * kSegRows + i;
    if (row >= count) break;
    const int64_t pool_row = slot * a.pool_rows + offset + row;
    const int64_t batch_row = start + row;
    const int64_t s = (GATHER ? pool_row : batch_row) * a.src_stride;
    const int64_t d = (GATHER ? batch_row : pool_row) * a.dst_stride;
    reinterpret_cast<raw_t*>(a.dst + d)[j] = reinterpret_cast<const raw_t*>(a.src + s)[j];
  }
}

template <int VB>
__global__ __launch_bounds__(kThreads) void gather_segments_kernel(SegmentArgs a) {
  segments_body<VB, true>(a);
}
template <int VB>
__global__ __launch_bounds__(kThreads) void scatter_segments_kernel(SegmentArgs a) {
  segments_body<VB, false>(a);
}

int launch_rows(bool gather, const void* src, void* dst, const int64_t* slots, int64_t n,
                int64_t rows, int64_t width, int64_t src_stride, int64_t dst_stride,
                hipStream_t s, const char* who) {
  VRH_CHECK_ARG(rows >= 0 && n >= 0 && width >= 0, "%s: negative size", who);
  if (rows == 0 || width == 0) return VRH_OK;
  VRH_CHECK_ARG(src && dst && slots, "%s: null pointer", who);
  VRH_CHECK_ARG(src_stride >= width && dst_stride >= width, "%s: row stride below width", who);
  const int vb = pick_vb({width, src_stride, dst_stride}, {src, dst});
  RowsArgs a;
  a.src = static_cast<const char*>(src);
  a.dst = static_cast<char*>(dst);
  a.slots = slots;
  a.n = n;
  a.vecs = width / vb;
  a.src_stride = src_stride;
  a.dst_stride = dst_stride;
  const int64_t gx = ceil_div64(a.vecs, kThreads);
  VRH_CHECK_ARG(gx < (1ll << 31), "%s: rows too wide", who);
  for (int64_t first = 0; first < rows; first += kMaxGrid) {
    a.row_base = first;
    const dim3 grid((unsigned)gx, (unsigned)std::min(rows - first, kMaxGrid));
    if (gather) VRH_DISPATCH_VB(vb, gather_rows_kernel, grid, dim3(kThreads), s, a)
    else VRH_DISPATCH_VB(vb, scatter_rows_kernel, grid, dim3(kThreads), s, a)
  }
  VRH_RETURN_LAUNCH(who);
}

int launch_segments(bool gather, const void* src, void* dst, const int64_t* segments,
                    int64_t num_segments, int64_t max_rows, int64_t pool_rows, int64_t width,
                    int64_t src_stride, int64_t dst_stride, hipStream_t s, const char* who) {
  VRH_CHECK_ARG(num_segments >= 0 && max_rows >= 0 && pool_rows >= 0 && width >= 0,
                "%s: negative size", who);
  if (num_segments == 0 || max_rows == 0 || width == 0) return VRH_OK;
  VRH_CHECK_ARG(src && dst && segments, "%s: null pointer", who);
  VRH_CHECK_ARG(src_stride >= width && dst_stride >= width, "%s: row stride below width", who);
  const int vb = pick_vb({width, src_stride, dst_stride}, {src, dst});
  SegmentArgs a;
  a.src = static_cast<const char*>(src);
  a.dst = static_cast<char*>(dst);
  a.segments = segments;
  a.pool_rows = pool_rows;
  a.vecs = width / vb;
  a.src_stride = src_stride;
  a.dst_stride = dst_stride;
  const int64_t gx = ceil_div64(a.vecs, kThreads);
  const int64_t gy = ceil_div64(max_rows, kSegRows);
  VRH_CHECK_ARG(gx < (1ll << 31) && gy <= kMaxGrid, "%s: segment too large", who);
  for (int64_t first = 0; first < num_segments; first += kMaxGrid) {
    a.seg_base = first;
    const dim3 grid((unsigned)gx, (unsigned)gy, (unsigned)std::min(num_segments - first, kMaxGrid));
    if (gather) VRH_DISPATCH_VB(vb, gather_segments_kernel, grid, dim3(kThreads), s, a)
    else VRH_DISPATCH_VB(vb, scatter_segments_kernel, grid, dim3(kThreads), s, a)
  }
  VRH_RETURN_LAUNCH(who);
}

}  // namespace
}  // namespace vrh

using namespace vrh;

extern "C" int vrh_gather_rows(const void* pool, const int64_t* slots, void* out, int64_t n,
                               int64_t size, int64_t width_bytes, int64_t pool_stride_bytes,
                               int64_t out_stride_bytes, vrh_stream_t stream) {
  return launch_rows(true, pool, out, slots, n, size, width_bytes, pool_stride_bytes,
                     out_stride_bytes, (hipStream_t)stream, "vrh_gather_rows");
}

extern "C" int vrh_scatter_rows(const void* in, const int64_t* slots, void* pool, int64_t count,
                                int64_t width_bytes, int64_t in_stride_bytes,
                                int64_t pool_stride_bytes, vrh_stream_t stream) {
  return launch_rows(false, in, pool, slots, count, count, width_bytes, in_stride_bytes,
                     pool_stride_bytes, (hipStream_t)stream, "vrh_scatter_rows");
}

extern "C" int vrh_gather_segments(const void* pool, const int64_t* segments, void* out,
                                   int64_t num_segments, int64_t max_rows, int64_t pool_rows,
                                   int64_t width_bytes, int64_t pool_stride_bytes,
                                   int64_t out_stride_bytes, vrh_stream_t stream) {
  return launch_segments(true, pool, out, segments, num_segments, max_rows, pool_rows,
                         width_bytes, pool_stride_bytes, out_stride_bytes, (hipStream_t)stream,
                         "vrh_gather_segments");
}

extern "C" int vrh_scatter_segments(const void* in, const int64_t* segments, void* pool,
                                    int64_t num_segments, int64_t max_rows, int64_t pool_rows,
                                    int64_t width_bytes, int64_t in_stride_bytes,
                                    int64_t pool_stride_bytes, vrh_stream_t stream) {
  return launch_segments(false, in, pool, segments, num_segments, max_rows, pool_rows,
                         width_bytes, in_stride_bytes, pool_stride_bytes, (hipStream_t)stream,
                         "vrh_scatter_segments");
}
