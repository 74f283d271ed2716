// Torch operator registration over the C ABI (libvllm_rlt_hip.so).
//
// Built as the Python extension module `vllm_rlt._C`, the module the
// reference's loader imports (kernels/_extension.py:7-23). Importing it
// registers, through TORCH_LIBRARY as the reference's csrc/torch_bindings.cpp:6-14
// does:
//   vllm_rlt::silu_and_mul      the reference's own op and schema (its native
//                               entry: csrc/activation/silu_and_mul.cu:221-245)
//   vllm_rlt_hip::paged_attention, paged_prefill, kv_append, kv_gather,
//                 kv_finalize, kv_copy_blocks
//                               the paged KV hot path, with the argument
//                               meaning of vllm_rlt/kernels/hip_attention.py
// Each op checks its tensors with TORCH_CHECK (RuntimeError), allocates
// outputs and workspaces through PyTorch's caching allocator, launches on the
// current stream of the tensors' device and forwards raw pointers and strides
// to the C entry point; a failing entry point raises with its message. Only
// the CUDA dispatch key (ROCm devices) has kernels.
#include <Python.h>

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "vllm_rlt_hip.h"

namespace {

int dtype_code(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return VRH_DTYPE_F32;
    case at::kHalf: return VRH_DTYPE_F16;
    case at::kBFloat16: return VRH_DTYPE_BF16;
    default: TORCH_CHECK(false, "the hip backend supports float32, float16 and bfloat16, not ",
                         t.scalar_type());
  }
}

vrh_stream_t stream_of(const at::Tensor& t) {
  return reinterpret_cast<vrh_stream_t>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_rc(int rc, const char* who) {
  TORCH_CHECK(rc == VRH_OK, who, ": ", vrh_last_error());
}

void check_gpu(const char* name, const at::Tensor& t, const at::Device& device) {
  TORCH_CHECK(t.is_cuda(), name, " must be a ROCm device tensor for the hip backend");
  TORCH_CHECK(t.device() == device, name, " is on ", t.device(), ", expected ", device);
}

void check_int(const char* name, const at::Tensor& t, at::ScalarType dtype, int64_t ndim,
               const at::Device& device) {
  check_gpu(name, t, device);
  TORCH_CHECK(t.scalar_type() == dtype && t.dim() == ndim, name, " must be a ", ndim, "-D ",
              dtype, " tensor");
}

// q [rows, Hq, D] and one layer view [blocks, block_size, Hkv, D] of each cache.
void check_attention(const at::Tensor& q, const at::Tensor& kc, const at::Tensor& vc,
                     const at::Tensor& tables, const at::Tensor& lengths) {
  TORCH_CHECK(q.dim() == 3, "q must be [rows, q_heads, head_dim]");
  dtype_code(q);
  check_gpu("q", q, q.device());
  for (const auto* c : {&kc, &vc}) {
    const char* name = c == &kc ? "key_cache" : "value_cache";
    check_gpu(name, *c, q.device());
    TORCH_CHECK(c->dim() == 4, name, " must be [blocks, block_size, kv_heads, head_dim]");
    TORCH_CHECK(c->scalar_type() == q.scalar_type(), name, " dtype differs from the query dtype");
    TORCH_CHECK(c->size(3) == q.size(2), name, " head_dim differs from the query head_dim");
    TORCH_CHECK(c->stride(3) == 1, name, " must have a contiguous head dimension");
  }
  TORCH_CHECK(vc.sizes() == kc.sizes(), "key_cache and value_cache shapes differ");
  TORCH_CHECK(q.size(1) > 0 && q.size(1) % kc.size(2) == 0,
              "query heads must be a positive multiple of KV heads");
  check_int("block_tables", tables, at::kInt, 2, q.device());
  check_int("context_lengths", lengths, at::kInt, 1, q.device());
  TORCH_CHECK(tables.size(1) == 0 || tables.stride(1) == 1, "block_tables rows must be contiguous");
}

at::Tensor paged_attention(const at::Tensor& q_in, const at::Tensor& kc, const at::Tensor& vc,
                           const at::Tensor& tables, const at::Tensor& lengths_in,
                           int64_t window) {
  TORCH_CHECK(window >= 0, "window must be a nonnegative integer");
  check_attention(q_in, kc, vc, tables, lengths_in);
  const at::Tensor q = q_in.stride(2) == 1 ? q_in : q_in.contiguous();
  const at::Tensor lengths = lengths_in.contiguous();
  const int64_t rows = q.size(0);
  TORCH_CHECK(tables.size(0) == rows && lengths.size(0) == rows,
              "block_tables and context_lengths must have one row per query row");
  const c10::DeviceGuard guard(q.device());
  at::Tensor out = at::empty_like(q);
  if (rows == 0) return out;
  const int32_t heads = (int32_t)q.size(1), dim = (int32_t)q.size(2);
  const size_t nbytes = vrh_paged_decode_workspace_bytes(rows, heads, dim);
  at::Tensor workspace = at::empty({(int64_t)nbytes}, q.options().dtype(at::kByte));
  check_rc(vrh_paged_decode(dtype_code(q), out.data_ptr(), q.data_ptr(), kc.data_ptr(),
                            vc.data_ptr(), tables.data_ptr<int32_t>(), lengths.data_ptr<int32_t>(),
                            rows, heads, (int32_t)kc.size(2), dim, (int32_t)kc.size(1),
                            (int32_t)tables.size(1), tables.stride(0), q.stride(0), q.stride(1),
                            out.stride(0), out.stride(1), kc.stride(0), kc.stride(1), kc.stride(2),
                            vc.stride(0), vc.stride(1), vc.stride(2), (int32_t)window,
                            workspace.data_ptr(), nbytes, stream_of(q)),
           "vrh_paged_decode");
  return out;
}

at::Tensor paged_prefill(const at::Tensor& q_in, const at::Tensor& kc, const at::Tensor& vc,
                         const at::Tensor& tables, const at::Tensor& lengths_in,
                         const at::Tensor& cu_in, int64_t max_seqlen_q) {
  check_attention(q_in, kc, vc, tables, lengths_in);
  check_int("cu_seqlens_q", cu_in, at::kInt, 1, q_in.device());
  const at::Tensor q = q_in.stride(2) == 1 ? q_in : q_in.contiguous();
  const at::Tensor lengths = lengths_in.contiguous();
  const at::Tensor cu = cu_in.contiguous();
  const int64_t seqs = tables.size(0);
  TORCH_CHECK(lengths.size(0) == seqs && cu.size(0) == seqs + 1,
              "prefill metadata must describe the same number of sequences");
  TORCH_CHECK(max_seqlen_q >= 0 && max_seqlen_q < (1ll << 31), "max_seqlen_q out of range");
  const c10::DeviceGuard guard(q.device());
  at::Tensor out = at::empty_like(q);
  if (q.size(0) == 0 || seqs == 0) return out;
  const int32_t heads = (int32_t)q.size(1), dim = (int32_t)q.size(2);
  const size_t nbytes = vrh_paged_prefill_workspace_bytes(seqs, (int32_t)max_seqlen_q, heads, dim);
  at::Tensor workspace = at::empty({(int64_t)nbytes}, q.options().dtype(at::kByte));
  check_rc(vrh_paged_prefill(dtype_code(q), out.data_ptr(), q.data_ptr(), kc.data_ptr(),
                             vc.data_ptr(), tables.data_ptr<int32_t>(),
                             lengths.data_ptr<int32_t>(), cu.data_ptr<int32_t>(), seqs, q.size(0),
                             (int32_t)max_seqlen_q, heads, (int32_t)kc.size(2), dim,
                             (int32_t)kc.size(1), (int32_t)tables.size(1), tables.stride(0),
                             q.stride(0), q.stride(1), out.stride(0), out.stride(1), kc.stride(0),
                             kc.stride(1), kc.stride(2), vc.stride(0), vc.stride(1), vc.stride(2),
                             workspace.data_ptr(), nbytes, stream_of(q)),
           "vrh_paged_prefill");
  return out;
}

// One layer view [blocks, block_size, Hkv, D] of each cache; k, v [rows, Hkv, D].
void kv_append(const at::Tensor& kc, const at::Tensor& vc, const at::Tensor& k,
               const at::Tensor& v, const at::Tensor& blocks_in, const at::Tensor& offsets_in,
               const std::optional<at::Tensor>& mask, const std::optional<at::Tensor>& active) {
  dtype_code(kc);
  const at::Device device = kc.device();
  check_gpu("key_cache", kc, device);
  check_gpu("value_cache", vc, device);
  TORCH_CHECK(kc.dim() == 4 && vc.sizes() == kc.sizes(),
              "caches must be matching [blocks, block_size, kv_heads, head_dim] views");
  TORCH_CHECK(kc.strides() == vc.strides(), "key_cache and value_cache must share strides");
  TORCH_CHECK(kc.stride(3) == 1, "caches must have a contiguous head dimension");
  for (const auto* t : {&k, &v}) {
    const char* name = t == &k ? "k" : "v";
    check_gpu(name, *t, device);
    TORCH_CHECK(t->scalar_type() == kc.scalar_type(), name, " must use the cache dtype");
    TORCH_CHECK(t->dim() == 3 && t->size(1) == kc.size(2) && t->size(2) == kc.size(3), name,
                " must be [rows, ", kc.size(2), ", ", kc.size(3), "]");
    TORCH_CHECK(t->stride(2) == 1, name, " must have a contiguous head dimension");
  }
  const int64_t rows = k.size(0);
  TORCH_CHECK(v.size(0) == rows, "k and v must have the same rows");
  check_int("write_blocks", blocks_in, at::kLong, 1, device);
  check_int("write_offsets", offsets_in, at::kLong, 1, device);
  TORCH_CHECK(blocks_in.size(0) >= rows && offsets_in.size(0) >= rows,
              "write_blocks and write_offsets need an entry per row");
  at::Tensor mask_c;
  if (mask.has_value()) {
    check_int("write_mask", *mask, at::kBool, 1, device);
    TORCH_CHECK(mask->size(0) >= rows, "write_mask needs an entry per row");
    mask_c = mask->contiguous();
  }
  if (active.has_value()) {
    check_gpu("active_rows", *active, device);
    TORCH_CHECK(active->scalar_type() == at::kInt && active->numel() == 1,
                "active_rows must be a device int32 scalar");
  }
  if (rows == 0) return;
  const c10::DeviceGuard guard(device);
  const at::Tensor blocks = blocks_in.contiguous(), offsets = offsets_in.contiguous();
  check_rc(vrh_kv_append(dtype_code(kc), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
                         kc.stride(2), 0, k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), 0,
                         v.stride(0), v.stride(1), 0, blocks.data_ptr<int64_t>(),
                         offsets.data_ptr<int64_t>(),
                         mask.has_value() ? reinterpret_cast<const uint8_t*>(mask_c.data_ptr())
                                          : nullptr,
                         active.has_value() ? active->data_ptr<int32_t>() : nullptr, rows, 1,
                         (int32_t)kc.size(2), (int32_t)kc.size(3), kc.size(0),
                         (int32_t)kc.size(1), stream_of(kc)),
           "vrh_kv_append");
}

// Byte strides of a cache whose (kv_heads, head_dim) token slot is dense.
int64_t slot_bytes(const at::Tensor& c, const char* name) {
  const int64_t nd = c.dim();
  TORCH_CHECK(c.stride(nd - 1) == 1 && c.stride(nd - 2) == c.size(nd - 1), name,
              " token slots must be contiguous [kv_heads, head_dim]");
  return c.size(nd - 2) * c.size(nd - 1) * c.element_size();
}

std::tuple<at::Tensor, at::Tensor> kv_gather(const at::Tensor& kc, const at::Tensor& vc,
                                             const at::Tensor& table_in, int64_t length) {
  check_gpu("key_cache", kc, kc.device());
  check_gpu("value_cache", vc, kc.device());
  check_int("table", table_in, at::kInt, 1, kc.device());
  TORCH_CHECK(kc.dim() == 4 && kc.sizes() == vc.sizes() && kc.strides() == vc.strides(),
              "key_cache and value_cache must match");
  const int64_t channel = slot_bytes(kc, "key_cache");
  const int64_t bs = kc.size(1);
  TORCH_CHECK(length >= 0 && (length + bs - 1) / bs <= table_in.size(0),
              "length exceeds the table");
  const c10::DeviceGuard guard(kc.device());
  at::Tensor keys = at::empty({length, kc.size(2), kc.size(3)}, kc.options());
  at::Tensor values = at::empty_like(keys);
  if (length == 0) return {keys, values};
  const at::Tensor table = table_in.contiguous();
  const int64_t es = kc.element_size();
  check_rc(vrh_kv_gather(keys.data_ptr(), values.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                         table.data_ptr<int32_t>(), length, (int32_t)bs, kc.stride(0) * es,
                         kc.stride(1) * es, channel, stream_of(kc)),
           "vrh_kv_gather");
  return {keys, values};
}

// Whole pools [blocks, layers, block_size, Hkv, D].
void check_pools(const at::Tensor& kc, const at::Tensor& vc) {
  check_gpu("key_cache", kc, kc.device());
  check_gpu("value_cache", vc, kc.device());
  TORCH_CHECK(kc.dim() == 5 && vc.sizes() == kc.sizes(), "caches must be matching 5-D pools");
  TORCH_CHECK(kc.strides() == vc.strides(), "key_cache and value_cache must share strides");
}

void kv_finalize(const at::Tensor& kc, const at::Tensor& vc, const at::Tensor& desc_in,
                 const at::Tensor& tables_in, int64_t planes) {
  check_pools(kc, vc);
  check_int("descriptors", desc_in, at::kLong, 2, kc.device());
  check_int("tables", tables_in, at::kInt, 2, kc.device());
  TORCH_CHECK(desc_in.size(1) == 3, "descriptors must be [rows, 3] (slot, depth, position)");
  const int64_t channel = slot_bytes(kc, "key_cache");
  const int64_t rows = desc_in.size(0);
  if (rows == 0 || planes <= 1) return;
  const c10::DeviceGuard guard(kc.device());
  const at::Tensor desc = desc_in.contiguous(), tables = tables_in.contiguous();
  const int64_t es = kc.element_size();
  check_rc(vrh_kv_finalize(kc.data_ptr(), vc.data_ptr(), desc.data_ptr<int64_t>(),
                           tables.data_ptr<int32_t>(), rows, (int32_t)planes,
                           (int32_t)tables.size(1), (int32_t)kc.size(2), (int32_t)kc.size(1),
                           kc.stride(0) * es, kc.stride(1) * es, kc.stride(2) * es, channel,
                           stream_of(kc)),
           "vrh_kv_finalize");
}

void kv_copy_blocks(const at::Tensor& kc, const at::Tensor& vc, const at::Tensor& src_in,
                    const at::Tensor& dst_in) {
  check_gpu("key_cache", kc, kc.device());
  check_gpu("value_cache", vc, kc.device());
  TORCH_CHECK(kc.dim() >= 2 && kc.sizes() == vc.sizes() && kc.strides() == vc.strides(),
              "key_cache and value_cache must match");
  check_int("src_blocks", src_in, at::kLong, 1, kc.device());
  check_int("dst_blocks", dst_in, at::kLong, 1, kc.device());
  TORCH_CHECK(src_in.size(0) == dst_in.size(0), "src_blocks and dst_blocks must have equal lengths");
  const int64_t n = src_in.size(0);
  if (n == 0) return;
  const at::Tensor block = kc[0];
  TORCH_CHECK(block.is_contiguous(), "each pool block must be contiguous");
  const c10::DeviceGuard guard(kc.device());
  const at::Tensor src = src_in.contiguous(), dst = dst_in.contiguous();
  const int64_t es = kc.element_size();
  check_rc(vrh_kv_copy_blocks(kc.data_ptr(), vc.data_ptr(), kc.stride(0) * es,
                              block.numel() * es, src.data_ptr<int64_t>(),
                              dst.data_ptr<int64_t>(), n, stream_of(kc)),
           "vrh_kv_copy_blocks");
}

// The reference's native entry, same checks and messages.
at::Tensor silu_and_mul(const at::Tensor& gate, const at::Tensor& up) {
  TORCH_CHECK(gate.is_cuda() && up.is_cuda(), "silu_and_mul expects CUDA inputs");
  TORCH_CHECK(gate.device() == up.device(), "silu_and_mul expects inputs on the same device");
  TORCH_CHECK(gate.sizes() == up.sizes(), "silu_and_mul expects inputs with the same shape");
  TORCH_CHECK(gate.scalar_type() == up.scalar_type(),
              "silu_and_mul expects inputs with the same dtype");
  TORCH_CHECK(gate.scalar_type() == at::kFloat || gate.scalar_type() == at::kHalf ||
                  gate.scalar_type() == at::kBFloat16,
              "silu_and_mul supports float32, float16 and bfloat16");
  TORCH_CHECK(gate.is_contiguous() && up.is_contiguous(), "silu_and_mul expects contiguous inputs");
  TORCH_CHECK(!at::GradMode::is_enabled() || (!gate.requires_grad() && !up.requires_grad()),
              "silu_and_mul is inference-only; use torch.no_grad() or silu_and_mul_reference");
  const c10::DeviceGuard guard(gate.device());
  at::Tensor out = at::empty(gate.sizes(), gate.options());
  if (gate.numel() == 0) return out;
  check_rc(vrh_silu_and_mul(dtype_code(gate), out.data_ptr(), gate.data_ptr(), up.data_ptr(),
                            gate.numel(), stream_of(gate)),
           "vrh_silu_and_mul");
  return out;
}

}  // namespace

TORCH_LIBRARY(vllm_rlt, ops) {
  ops.def("silu_and_mul(Tensor gate, Tensor up) -> Tensor");
}

TORCH_LIBRARY_IMPL(vllm_rlt, CUDA, ops) {
  ops.impl("silu_and_mul", &silu_and_mul);
}

TORCH_LIBRARY(vllm_rlt_hip, ops) {
  ops.def("paged_attention(Tensor q, Tensor key_cache, Tensor value_cache, Tensor block_tables, "
          "Tensor context_lengths, int window=0) -> Tensor");
  ops.def("paged_prefill(Tensor q, Tensor key_cache, Tensor value_cache, Tensor block_tables, "
          "Tensor context_lengths, Tensor cu_seqlens_q, int max_seqlen_q) -> Tensor");
  ops.def("kv_append(Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor k, Tensor v, "
          "Tensor write_blocks, Tensor write_offsets, Tensor? write_mask=None, "
          "Tensor? active_rows=None) -> ()");
  ops.def("kv_gather(Tensor key_cache, Tensor value_cache, Tensor table, int length) "
          "-> (Tensor, Tensor)");
  ops.def("kv_finalize(Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor descriptors, "
          "Tensor tables, int planes) -> ()");
  ops.def("kv_copy_blocks(Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor src_blocks, "
          "Tensor dst_blocks) -> ()");
}

TORCH_LIBRARY_IMPL(vllm_rlt_hip, CUDA, ops) {
  ops.impl("paged_attention", &paged_attention);
  ops.impl("paged_prefill", &paged_prefill);
  ops.impl("kv_append", &kv_append);
  ops.impl("kv_gather", &kv_gather);
  ops.impl("kv_finalize", &kv_finalize);
  ops.impl("kv_copy_blocks", &kv_copy_blocks);
}

// An empty Python module: importing it runs the registrations above.
static PyModuleDef vrh_module = {PyModuleDef_HEAD_INIT, "_C", nullptr, -1, nullptr};
PyMODINIT_FUNC PyInit__C(void) { return PyModule_Create(&vrh_module); }
