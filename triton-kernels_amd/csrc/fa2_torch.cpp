// fa2_torch.cpp - the launch half of flash_attention_v2 / flash_attention_v1
// as a PyTorch-ROCm extension: after the Python wrapper has run the
// reference's assertion sequence (kernels/attention.py mirrors
// attention.py:762-834), one call here derives the sizes of the layout,
// makes rows 16-byte aligned, converts the index tensors, allocates the
// output and the workspace from torch's caching allocator, fills
// fa2_params and enqueues fa2_fwd (include/fa2.h) on torch's current HIP
// stream.  It replaces a chain of Python steps (strides, pointer fields,
// a ctypes call) that cost ~11 us per call, more than small calls take on
// the GPU.  No attention arithmetic here.
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include "fa2.h"

namespace {

// Last dim contiguous and every row start 16-byte aligned (the kernels'
// requirement; kernels/_launch.py:rows_ok).
bool rows_ok(const at::Tensor& t) {
  if (t.numel() == 0) return true;
  const int64_t es = t.element_size();
  const auto addr = reinterpret_cast<uintptr_t>(t.data_ptr());
  if (t.is_contiguous()) return addr % 16 == 0 && (t.size(-1) * es) % 16 == 0;
  if (t.stride(-1) != 1 || addr % 16) return false;
  for (int64_t d = 0; d + 1 < t.dim(); ++d)
    if ((t.stride(d) * es) % 16) return false;
  return true;
}

at::Tensor prep(const at::Tensor& t) { return rows_ok(t) ? t : t.contiguous(); }

// (batch, head, row) element strides; token-major tensors (token, head).
void strides3(const at::Tensor& t, int64_t& sb, int64_t& sh, int64_t& ss) {
  if (t.dim() == 4) {
    sb = t.stride(0);
    sh = t.stride(1);
    ss = t.stride(2);
  } else {
    sb = 0;
    sh = t.stride(1);
    ss = t.stride(0);
  }
}

at::Tensor index32(const at::Tensor& t, const at::Device& dev) {
  if (t.scalar_type() != at::kInt || !t.is_contiguous() || t.device() != dev)
    return t.to(dev, at::kInt).contiguous();
  return t;
}

at::Tensor table32(const at::Tensor& t, const at::Device& dev) {
  if (t.scalar_type() != at::kInt || t.stride(-1) != 1 || t.device() != dev)
    return t.to(dev, at::kInt).contiguous();
  return t;
}

int32_t dtype_code(at::ScalarType s) {
  switch (s) {
    case at::kHalf: return FA2_DTYPE_F16;
    case at::kBFloat16: return FA2_DTYPE_BF16;
    default: return FA2_DTYPE_F32;
  }
}

// layout: FA2_LAYOUT_*; mask: FA2_MASK_*; the tensors have passed the
// wrapper's asserts and dtype / head-dim checks.
at::Tensor fwd(at::Tensor q, at::Tensor k, at::Tensor v, int64_t layout, int64_t mask,
               c10::optional<at::Tensor> q_indptr, c10::optional<at::Tensor> kv_indptr,
               c10::optional<at::Tensor> k_block_table, c10::optional<at::Tensor> v_block_table,
               int64_t page_size, int64_t num_splits, int64_t max_workgroups, int64_t arith,
               int64_t kernel) {
  const at::Device dev = q.device();
  const c10::DeviceGuard guard(dev);
  fa2_params p;
  std::memset(&p, 0, sizeof(p));
  p.layout = static_cast<int32_t>(layout);
  p.dtype = dtype_code(q.scalar_type());
  p.mask = static_cast<int32_t>(mask);
  p.num_splits = static_cast<int32_t>(num_splits);
  p.max_workgroups = static_cast<int32_t>(max_workgroups);
  p.arith = static_cast<int32_t>(arith);
  p.kernel = static_cast<int32_t>(kernel);

  at::Tensor qi, kvi, kt, vt;
  if (layout == FA2_LAYOUT_DENSE) {
    p.batch = q.size(0);
    p.q_heads = q.size(1);
    p.q_len = q.size(2);
    p.head_dim = q.size(3);
    p.kv_heads = k.size(1);
    p.kv_len = k.size(2);
  } else if (layout == FA2_LAYOUT_RAGGED) {
    qi = index32(*q_indptr, dev);
    kvi = index32(*kv_indptr, dev);
    p.batch = q_indptr->numel() - 1;
    p.q_heads = q.size(1);
    p.q_len = q.size(0);
    p.head_dim = q.size(2);
    p.kv_heads = k.size(1);
    p.kv_len = k.size(0);
  } else {
    kvi = index32(*kv_indptr, dev);
    kt = table32(*k_block_table, dev);
    vt = table32(*v_block_table, dev);
    p.batch = q.size(0);
    p.q_heads = q.size(1);
    p.q_len = q.size(2);
    p.head_dim = q.size(3);
    p.kv_heads = k.size(1);
    p.kv_len = k.size(0);  // the caches' rows
    p.page_size = page_size;
    p.kv_len_max = k_block_table->size(1) * page_size;  // the reference's N (:834)
    p.k_table_stride = kt.stride(0);
    p.v_table_stride = vt.stride(0);
  }
  p.softmax_scale = static_cast<float>(std::pow(static_cast<double>(p.head_dim), -0.5));  // D ** -0.5 (:897)

  q = prep(q);
  k = prep(k);
  v = prep(v);
  at::Tensor out = at::empty_like(q);  // contiguous and aligned when q is
  if (!q.is_contiguous() && !rows_ok(out)) out = at::empty(q.sizes(), q.options());

  strides3(q, p.q_sb, p.q_sh, p.q_ss);
  strides3(k, p.k_sb, p.k_sh, p.k_ss);
  strides3(v, p.v_sb, p.v_sh, p.v_ss);
  strides3(out, p.o_sb, p.o_sh, p.o_ss);
  p.q = q.data_ptr();
  p.k = k.data_ptr();
  p.v = v.data_ptr();
  p.o = out.data_ptr();
  if (qi.defined()) p.q_indptr = qi.data_ptr<int32_t>();
  if (kvi.defined()) p.kv_indptr = kvi.data_ptr<int32_t>();
  if (kt.defined()) {
    p.k_block_table = kt.data_ptr<int32_t>();
    p.v_block_table = vt.data_ptr<int32_t>();
  }

  size_t ws_bytes = 0;
  int rc = fa2_fwd_workspace_size(&p, &ws_bytes);
  TORCH_CHECK(rc == FA2_OK, "flash_attention_v2: ", fa2_strerror(rc), " (fa2 status ", rc, ")");
  at::Tensor ws;
  if (ws_bytes) {
    ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
    p.workspace = ws.data_ptr();
    p.workspace_bytes = ws_bytes;
  }
  const hipStream_t st = c10::hip::getCurrentHIPStream(dev.index()).stream();
  rc = fa2_fwd(&p, st);
  TORCH_CHECK(rc == FA2_OK, "flash_attention_v2: ", fa2_strerror(rc), " (fa2 status ", rc, ")");
  return out;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("fwd", &fwd, "enqueue fa2_fwd for checked tensors; returns the output");
}
