// Paged decode without any device allocation: the split partials live in a
// file-scope device array instead of a caller workspace.
//
// For callers that cannot allocate (code under HIP-graph capture that must not
// grow a pool, tight serving loops, harnesses that forbid hipMalloc). The
// kernels are the ones of vrh_paged_decode; only the partials' home differs.
//
// `scratch` is one array per GPU: 96 MiB of device memory reserved on every
// GPU where this library's code object is loaded, whether or not the entry
// point is ever called, and held until the process ends. Its address is
// looked up once per device (hipGetSymbolAddress with that device current, at
// the first vrh_paged_decode_noalloc_max_bytes or vrh_paged_decode_noalloc
// call on it) and kept; host code never passes the array's name itself to a kernel (on the
// host that name is only a stand-in, not a device address). The partials need
// no initialisation: every split the merge reads is written by the same call
// first. Calls that overlap on one GPU (different streams, or graphs replayed
// concurrently) share the array and race.
#include <mutex>

#include "common.h"

int vrh_decode_rows(int dtype, void* out, const void* q, const void* key_cache,
                    const void* value_cache, const int32_t* block_tables,
                    const int32_t* context_lengths, const int32_t* cu_q, int32_t num_seqs,
                    int32_t expand_e, int64_t rows, int32_t q_heads, int32_t kv_heads,
                    int32_t head_dim, int32_t block_size, int32_t table_width,
                    int64_t table_stride, int64_t q_row_stride, int64_t q_head_stride,
                    int64_t out_row_stride, int64_t out_head_stride, int64_t k_block_stride,
                    int64_t k_token_stride, int64_t k_head_stride, int64_t v_block_stride,
                    int64_t v_token_stride, int64_t v_head_stride, int32_t window,
                    void* workspace, size_t workspace_bytes, hipStream_t s, const char* who);

static __device__ __align__(256) unsigned char scratch[VRH_PAGED_DECODE_NOALLOC_MAX_BYTES];

namespace {

constexpr size_t kScratchBytes = VRH_PAGED_DECODE_NOALLOC_MAX_BYTES;
constexpr int kMaxDevices = 64;

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// Device address of the current device's `scratch`, or nullptr (error set).
void* scratch_address(const char* who) {
  int device = -1;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess || device < 0 || device >= kMaxDevices) {
    vrh_set_error("%s: no usable current device (%s)", who,
                  e != hipSuccess ? hipGetErrorString(e) : "device index out of range");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      vrh_set_error("%s: hipGetSymbolAddress of the scratch array failed on device %d: %s", who,
                    device, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[device] = ptr;
  }
  return g_scratch_ptr[device];
}

}  // namespace

// Also looks up the current device's scratch address, so that a caller can do
// that before capturing a graph (the lookup is a runtime call, not a stream
// operation, and is done at most once per device). A failed lookup is
// reported by the first vrh_paged_decode_noalloc call instead.
extern "C" size_t vrh_paged_decode_noalloc_max_bytes(void) {
  scratch_address("vrh_paged_decode_noalloc_max_bytes");
  return kScratchBytes;
}

extern "C" int vrh_paged_decode_noalloc(
    int dtype, void* out, const void* q, const void* key_cache, const void* value_cache,
    const int32_t* block_tables, const int32_t* context_lengths, int64_t rows, int32_t q_heads,
    int32_t kv_heads, int32_t head_dim, int32_t block_size, int32_t table_width,
    int64_t table_stride, int64_t q_row_stride, int64_t q_head_stride, int64_t out_row_stride,
    int64_t out_head_stride, int64_t k_block_stride, int64_t k_token_stride,
    int64_t k_head_stride, int64_t v_block_stride, int64_t v_token_stride, int64_t v_head_stride,
    int32_t window, vrh_stream_t stream) {
  static const char* who = "vrh_paged_decode_noalloc";
  if (rows == 0) return VRH_OK;
  const size_t need = vrh_paged_decode_workspace_bytes(rows, q_heads, head_dim);
  VRH_CHECK_ARG(need <= kScratchBytes,
                "%s: %lld rows x %d heads x head_dim %d need %zu bytes of split partials; the "
                "built-in scratch holds %zu (use vrh_paged_decode with a workspace)",
                who, (long long)rows, q_heads, head_dim, need, kScratchBytes);
  void* ptr = scratch_address(who);
  if (ptr == nullptr) return VRH_ERROR_LAUNCH;
  return vrh_decode_rows(dtype, out, q, key_cache, value_cache, block_tables, context_lengths,
                         nullptr, 0, 0, rows, q_heads, kv_heads, head_dim, block_size, table_width,
                         table_stride, q_row_stride, q_head_stride, out_row_stride,
                         out_head_stride, k_block_stride, k_token_stride, k_head_stride,
                         v_block_stride, v_token_stride, v_head_stride, window, ptr, kScratchBytes,
                         (hipStream_t)stream, who);
}
