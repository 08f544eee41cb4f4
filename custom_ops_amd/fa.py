"""Op layer of ``recsys_ops::mha_fwd_with_mask`` on MI355X.

Mirrors the reference's torch op (Defyli/custom_ops):
  * schema ``mha_fwd_with_mask(Tensor q, Tensor k, Tensor v, Tensor mask) -> Tensor``
    (csrc/fa/fa_bindings.cpp:37-43, recsys.py:175-177), fake impl
    ``empty_like(q)`` (recsys.py:198-202);
  * validation order and messages of ``mha_fwd_with_mask_cuda``
    (csrc/fa/fa_fwd_op.cu:53-108) — every failure is a ``RuntimeError``;
  * CPU tensors are rejected like the reference's CPU stub
    (csrc/fa/fa_fwd_op.cu:199-207);
  * output ``empty_like(q)`` (fa_fwd_op.cu:141), scale 1/sqrt(d) (:186-188),
    launched on the current stream of q's device, no host sync (:191-194).

Differences by design: Sk % 8 != 0 needs no padded copies (fa_fwd_op.cu:117-134
pads K/V/mask); the HIP kernel predicates the tail in place. Split-KV partials
come from the caching allocator as one workspace tensor sized by the library.
"""
from __future__ import annotations

import math
import os

import torch

from . import _lib

NAMESPACE = "recsys_ops"
OP_NAME = "mha_fwd_with_mask"
SCHEMA = "mha_fwd_with_mask(Tensor q, Tensor k, Tensor v, Tensor mask) -> Tensor"


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def validate(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: torch.Tensor) -> None:
    """Input contract, in the reference's order (csrc/fa/fa_fwd_op.cu:53-108)."""
    _check(q.is_cuda, "q must be a CUDA tensor")
    _check(k.is_cuda, "k must be a CUDA tensor")
    _check(v.is_cuda, "v must be a CUDA tensor")
    _check(mask.is_cuda, "mask must be a CUDA tensor")
    _check(k.device == q.device and v.device == q.device and mask.device == q.device,
           "q, k, v and mask must be on the same device")

    is_fp16 = q.dtype == torch.float16
    is_bf16 = q.dtype == torch.bfloat16
    _check(is_fp16 or is_bf16, "q must be float16 or bfloat16")
    _check(k.dtype == q.dtype, "k dtype must match q")
    _check(v.dtype == q.dtype, "v dtype must match q")
    _check(mask.dtype == q.dtype, "mask dtype must match q")

    _check(q.is_contiguous(), "q must be contiguous")
    _check(k.is_contiguous(), "k must be contiguous")
    _check(v.is_contiguous(), "v must be contiguous")
    _check(mask.is_contiguous(), "mask must be contiguous")

    _check(q.dim() == 4, "q must be 4D (B, H, Sq, d)")
    _check(k.dim() == 4, "k must be 4D (B, Hk, Sk, d)")
    _check(v.dim() == 4, "v must be 4D (B, Hk, Sk, d)")
    _check(mask.dim() == 4, "mask must be 4D (B, 1, Sq, Sk)")

    B, H, Sq, d = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    _check(k.shape[0] == B and v.shape[0] == B and mask.shape[0] == B, "Batch size mismatch")
    _check(k.shape[3] == d and v.shape[3] == d, "head_dim mismatch between q/k/v")
    _check(k.shape[2] == Sk and v.shape[2] == Sk, "seqlen_k mismatch between k/v")
    _check(v.shape[1] == Hk, "n_kv_heads mismatch between k/v")
    _check(Hk > 0 and H % Hk == 0, "n_heads must be divisible by n_kv_heads (GQA)")
    _check(d in (64, 128), "Only head_dim=64 or head_dim=128 is supported")
    _check(mask.shape[1] == 1 and mask.shape[2] >= Sq and mask.shape[3] >= Sk,
           "mask shape must be (B, 1, >=Sq, k-dim >= Sk)")


def make_params(q, k, v, mask, out, num_splits: int = 0) -> _lib.Params:
    """Fill the C-ABI params (strides in elements) from validated tensors."""
    p = _lib.Params()
    p.q, p.k, p.v, p.mask, p.o = (q.data_ptr(), k.data_ptr(), v.data_ptr(), mask.data_ptr(),
                                  out.data_ptr())
    p.q_batch_stride, p.q_head_stride, p.q_row_stride = q.stride(0), q.stride(1), q.stride(2)
    p.k_batch_stride, p.k_head_stride, p.k_row_stride = k.stride(0), k.stride(1), k.stride(2)
    p.v_batch_stride, p.v_head_stride, p.v_row_stride = v.stride(0), v.stride(1), v.stride(2)
    p.o_batch_stride, p.o_head_stride, p.o_row_stride = out.stride(0), out.stride(1), out.stride(2)
    p.mask_batch_stride, p.mask_row_stride = mask.stride(0), mask.stride(2)
    p.b, p.h, p.seqlen_q, p.d = q.shape
    p.h_k, p.seqlen_k = k.shape[1], k.shape[2]
    p.mask_seqlen_q, p.mask_seqlen_k = mask.shape[2], mask.shape[3]
    p.dtype = _lib.BF16 if q.dtype == torch.bfloat16 else _lib.FP16
    p.scale_softmax = 1.0 / math.sqrt(q.shape[3])
    p.num_splits = num_splits
    return p


def mha_fwd_with_mask_hip(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          mask: torch.Tensor, num_splits: int = 0) -> torch.Tensor:
    """The device implementation (dispatch key CUDA = HIP on PyTorch-ROCm).

    ``num_splits`` = 0 lets the library's cost model choose; a positive value
    forces that many KV splits (tests use it to pin split invariance)."""
    validate(q, k, v, mask)
    out = torch.empty_like(q)
    if out.numel() == 0:
        return out
    p = make_params(q, k, v, mask, out, num_splits)
    with torch.cuda.device(q.device):
        ws_bytes = _lib.workspace_bytes(p)
        ws = None
        if ws_bytes:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
            p.workspace, p.workspace_bytes = ws.data_ptr(), ws_bytes
        stream = torch.cuda.current_stream(q.device).cuda_stream
        _lib.fwd(p, stream)
    # ws goes back to the caching allocator here; its reuse is ordered on this stream.
    del ws
    return out


def _cpu_impl(q, k, v, mask):
    raise RuntimeError("mha_fwd_with_mask is only supported on CUDA")


def _cuda_impl(q, k, v, mask):
    return mha_fwd_with_mask_hip(q, k, v, mask)


_registered = False
_torch_lib = None


def register() -> None:
    """Register recsys_ops::mha_fwd_with_mask with the dispatcher (idempotent)."""
    global _registered, _torch_lib
    if _registered:
        return
    lib = torch.library.Library(NAMESPACE, "FRAGMENT")
    lib.define(SCHEMA)
    lib.impl(OP_NAME, _cuda_impl, "CUDA")
    lib.impl(OP_NAME, _cpu_impl, "CPU")
    torch.library.register_fake(f"{NAMESPACE}::{OP_NAME}", lib=lib)(
        lambda q, k, v, mask: torch.empty_like(q))
    _torch_lib = lib
    _registered = True


def num_splits_for(q, k, v, mask) -> int:
    """The split count the library would use for these inputs (host query)."""
    validate(q, k, v, mask)
    out = torch.empty((0,), dtype=q.dtype, device=q.device)
    p = make_params(q, k, v, mask, out)
    p.o = q.data_ptr()
    with torch.cuda.device(q.device):
        return _lib.num_splits(p)


def env_num_splits() -> int | None:
    val = os.environ.get("MI355_FA_NUM_SPLITS")
    return int(val) if val and val.isdigit() and int(val) > 0 else None
