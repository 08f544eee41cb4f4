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
// Argument checks: the reference operator's checks, in its order and with its
// messages (csrc/fa/fa_fwd_op.cu:53-108), so callers see the same
// RuntimeError text through either binding. Two checks the reference does not
// make come after the ones it shares: all inputs on q's GPU, and k/v head
// counts equal (the C ABI carries one Hk, so a v with other heads would be
// read out of range). Everything shape-related is settled here, before any
// pointer reaches the library; mi355_fa_fwd then checks alignment and the
// 32-bit range limits of its buffer addressing.
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
  TORCH_CHECK(q.is_cuda(), "q must be a CUDA tensor");
  TORCH_CHECK(k.is_cuda(), "k must be a CUDA tensor");
  TORCH_CHECK(v.is_cuda(), "v must be a CUDA tensor");
  TORCH_CHECK(mask.is_cuda(), "mask must be a CUDA tensor");

  const bool is_fp16 = q.scalar_type() == at::kHalf;
  const bool is_bf16 = q.scalar_type() == at::kBFloat16;
  TORCH_CHECK(is_fp16 || is_bf16, "q must be float16 or bfloat16");
  TORCH_CHECK(k.scalar_type() == q.scalar_type(), "k dtype must match q");
  TORCH_CHECK(v.scalar_type() == q.scalar_type(), "v dtype must match q");
  TORCH_CHECK(mask.scalar_type() == q.scalar_type(), "mask dtype must match q");

  TORCH_CHECK(q.is_contiguous(), "q must be contiguous");
  TORCH_CHECK(k.is_contiguous(), "k must be contiguous");
  TORCH_CHECK(v.is_contiguous(), "v must be contiguous");
  TORCH_CHECK(mask.is_contiguous(), "mask must be contiguous");

  TORCH_CHECK(q.dim() == 4, "q must be 4D (B, H, Sq, d)");
  TORCH_CHECK(k.dim() == 4, "k must be 4D (B, Hk, Sk, d)");
  TORCH_CHECK(v.dim() == 4, "v must be 4D (B, Hk, Sk, d)");
  TORCH_CHECK(mask.dim() == 4, "mask must be 4D (B, 1, Sq, Sk)");

  const int64_t B = q.size(0), H = q.size(1), Sq = q.size(2), d = q.size(3);
  const int64_t Hk = k.size(1), Sk = k.size(2);
  TORCH_CHECK(k.size(0) == B && v.size(0) == B && mask.size(0) == B, "Batch size mismatch");
  TORCH_CHECK(k.size(3) == d && v.size(3) == d, "head_dim mismatch between q/k/v");
  TORCH_CHECK(k.size(2) == Sk && v.size(2) == Sk, "seqlen_k mismatch between k/v");
  TORCH_CHECK(Hk > 0 && H % Hk == 0, "n_heads must be divisible by n_kv_heads (GQA)");
  TORCH_CHECK(d == 64 || d == 128, "Only head_dim=64 or head_dim=128 is supported");
  TORCH_CHECK(mask.size(1) == 1 && mask.size(2) >= Sq && mask.size(3) >= Sk,
              "mask shape must be (B, 1, >=Sq, k-dim >= Sk)");

  // not in the reference (see the note at the top of this file)
  TORCH_CHECK(k.device() == q.device() && v.device() == q.device() && mask.device() == q.device(),
              "q, k, v and mask must be on the same device");
  TORCH_CHECK(v.size(1) == Hk, "n_kv_heads mismatch between k/v");

  c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  auto out = at::empty_like(q);
  if (out.numel() == 0) return out;
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
