// recsys_ops::mha_fwd_with_mask as a C++ torch extension over the C ABI of
// libmi355_fa.so: the binding a maintainer of the reference would add next to
// csrc/fa/fa_bindings.cpp (TORCH_LIBRARY_FRAGMENT + CUDA-key impl,
// fa_bindings.cpp:23-43), for PyTorch-ROCm. Built in-tree by
// custom_ops_amd.build as libmi355_fa_torch.so (linked to libmi355_fa.so next
// to it); loading it with torch.ops.load_library registers the operator with
// the reference's schema. This package's own Python shim (fa.py) registers
// the same operator through torch.library instead, so a process uses one or
// the other.
//
// Argument checks: the tensor properties the C ABI cannot see (device, rank,
// dtype agreement, innermost stride); shapes, GQA divisibility, alignment and
// the mask extent are checked by mi355_fa_fwd itself, whose error text is
// raised unchanged.
// PyTorch-ROCm presents GPUs as the "cuda" device type: the guard and the
// stream are the HIP ones that accept it (the *MasqueradingAsCUDA classes)
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <ATen/ATen.h>
#include <torch/library.h>

#include <cmath>

#include "mi355_fa.h"

namespace {

at::Tensor mha_fwd_with_mask_mi355(const at::Tensor& q, const at::Tensor& k,
                                      const at::Tensor& v, const at::Tensor& mask) {
  for (const at::Tensor* t : {&q, &k, &v, &mask}) {
    TORCH_CHECK(t->is_cuda() && t->device() == q.device(), "all inputs must be on the same GPU");
    TORCH_CHECK(t->dim() == 4, "q, k, v and mask must be 4-D");
    TORCH_CHECK(t->scalar_type() == q.scalar_type(), "q, k, v and mask must share one dtype");
  }
  TORCH_CHECK(q.scalar_type() == at::kBFloat16 || q.scalar_type() == at::kHalf,
              "q must be float16 or bfloat16");
  TORCH_CHECK(q.stride(3) == 1 && k.stride(3) == 1 && v.stride(3) == 1 && mask.stride(3) == 1,
              "the last dimension of q, k, v and mask must be contiguous");
  TORCH_CHECK(mask.size(0) == q.size(0) && mask.size(1) == 1, "mask must be (B, 1, >=Sq, >=Sk)");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q, q.options().memory_format(at::MemoryFormat::Contiguous));
  mi355_fa_params p{};
  p.q = q.data_ptr(); p.k = k.data_ptr(); p.v = v.data_ptr(); p.mask = mask.data_ptr();
  p.o = out.data_ptr();
  p.q_batch_stride = q.stride(0); p.q_head_stride = q.stride(1); p.q_row_stride = q.stride(2);
  p.k_batch_stride = k.stride(0); p.k_head_stride = k.stride(1); p.k_row_stride = k.stride(2);
  p.v_batch_stride = v.stride(0); p.v_head_stride = v.stride(1); p.v_row_stride = v.stride(2);
  p.o_batch_stride = out.stride(0); p.o_head_stride = out.stride(1); p.o_row_stride = out.stride(2);
  p.mask_batch_stride = mask.stride(0); p.mask_row_stride = mask.stride(2);
  p.b = (int)q.size(0); p.h = (int)q.size(1); p.h_k = (int)k.size(1);
  p.seqlen_q = (int)q.size(2); p.seqlen_k = (int)k.size(2);
  p.mask_seqlen_q = (int)mask.size(2); p.mask_seqlen_k = (int)mask.size(3); p.d = (int)q.size(3);
  p.dtype = q.scalar_type() == at::kBFloat16 ? MI355_FA_BF16 : MI355_FA_FP16;
  p.scale_softmax = 1.0f / std::sqrt((float)p.d);
  at::Tensor ws;   // split-KV partials, from the caching allocator
  if (const size_t n = mi355_fa_workspace_bytes(&p)) {
    ws = at::empty({(int64_t)n}, q.options().dtype(at::kByte));
    p.workspace = ws.data_ptr();
    p.workspace_bytes = n;
  }
  char err[512] = {0};
  const int rc = mi355_fa_fwd(&p, c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.device().index()).stream(), err, sizeof err);
  TORCH_CHECK(rc == MI355_FA_OK, err);
  return out;
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(recsys_ops, m) {
  m.def("mha_fwd_with_mask(Tensor q, Tensor k, Tensor v, Tensor mask) -> Tensor");
}
TORCH_LIBRARY_IMPL(recsys_ops, CUDA, m) { m.impl("mha_fwd_with_mask", &mha_fwd_with_mask_mi355); }
