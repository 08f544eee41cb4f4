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

Differences by design: Sk % 8 != 0 pads no K/V (fa_fwd_op.cu:117-134 pads
K/V/mask); the HIP kernels predicate the key tail in place, and a mask whose
rows are not 16-byte aligned is staged by a pre-pass into an aligned copy in
the workspace. Split-KV partials, the
live-tile map and the staged mask come from the caching allocator as one
workspace tensor sized by the library.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

NAMESPACE = "recsys_ops"
OP_NAME = "mha_fwd_with_mask"
SCHEMA = "mha_fwd_with_mask(Tensor q, Tensor k, Tensor v, Tensor mask) -> Tensor"


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


_HALF = (torch.float16, torch.bfloat16)


def _valid(q, k, v, mask) -> bool:
    """True exactly when every check of ``validate`` passes (one expression, no
    messages built), so the per-call path skips the ordered checks."""
    dt = q.dtype
    dev = q.get_device()
    if not (q.is_cuda and k.is_cuda and v.is_cuda and mask.is_cuda and dt in _HALF
            and k.dtype == dt and v.dtype == dt and mask.dtype == dt
            and k.get_device() == dev and v.get_device() == dev and mask.get_device() == dev
            and q.is_contiguous() and k.is_contiguous() and v.is_contiguous()
            and mask.is_contiguous()):
        return False
    qs, ks, vs, ms = q.shape, k.shape, v.shape, mask.shape
    if not (len(qs) == 4 and len(ks) == 4 and len(vs) == 4 and len(ms) == 4):
        return False
    B, H, Sq, d = qs
    Hk, Sk = ks[1], ks[2]
    return (ks[0] == B and vs[0] == B and ms[0] == B and ks[3] == d and vs[3] == d
            and vs[2] == Sk and vs[1] == Hk and Hk > 0 and H % Hk == 0 and d in (64, 128)
            and ms[1] == 1 and ms[2] >= Sq and ms[3] >= Sk)


def validate(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: torch.Tensor) -> None:
    """Input contract, in the reference's order and with its messages
    (csrc/fa/fa_fwd_op.cu:53-108), then two checks of this build's own. The
    C++ binding (csrc/torch_binding.cpp) makes the same checks in the same order."""
    if _valid(q, k, v, mask):
        return
    _check(q.is_cuda, "q must be a CUDA tensor")
    _check(k.is_cuda, "k must be a CUDA tensor")
    _check(v.is_cuda, "v must be a CUDA tensor")
    _check(mask.is_cuda, "mask must be a CUDA tensor")

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
    _check(Hk > 0 and H % Hk == 0, "n_heads must be divisible by n_kv_heads (GQA)")
    _check(d in (64, 128), "Only head_dim=64 or head_dim=128 is supported")
    _check(mask.shape[1] == 1 and mask.shape[2] >= Sq and mask.shape[3] >= Sk,
           "mask shape must be (B, 1, >=Sq, k-dim >= Sk)")
    # Not in the reference, which trusts both (the C ABI carries one Hk and
    # addresses every tensor on q's device): checked after the reference's own.
    _check(k.device == q.device and v.device == q.device and mask.device == q.device,
           "q, k, v and mask must be on the same device")
    _check(v.shape[1] == Hk, "n_kv_heads mismatch between k/v")


def make_params(q, k, v, mask, out, num_splits: int = 0, variant=None) -> _lib.Params:
    """Fill the C-ABI params (strides in elements) from validated tensors.
    ``variant`` (a ``_lib.Variant``) is referenced, not copied: keep it alive
    while the params are in use."""
    qs, ks, vs, os_, ms = q.stride(), k.stride(), v.stride(), out.stride(), mask.stride()
    B, H, Sq, d = q.shape
    p = _lib.Params(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), mask.data_ptr(), out.data_ptr(),
        qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2],
        os_[0], os_[1], os_[2], ms[0], ms[2],
        B, H, k.shape[1], Sq, k.shape[2], mask.shape[2], mask.shape[3], d,
        _lib.BF16 if q.dtype == torch.bfloat16 else _lib.FP16,
        1.0 / math.sqrt(d), num_splits)
    if variant is not None:
        p.variant = ctypes.pointer(variant)
    return p


def mha_fwd_with_mask_hip(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          mask: torch.Tensor, num_splits: int = 0, variant=None) -> torch.Tensor:
    """The device implementation (dispatch key CUDA = HIP on PyTorch-ROCm).

    ``num_splits`` = 0 lets the library plan the split; a positive value
    forces that many KV splits (tests use it to pin split invariance).
    ``variant`` (a ``_lib.Variant``, default None = the library's plan) forces
    kernel variants for parity tests and tuning."""
    validate(q, k, v, mask)
    out = torch.empty_like(q)
    if out.numel() == 0:
        return out
    p = make_params(q, k, v, mask, out, num_splits, variant)
    dev = q.get_device()
    if dev == torch.cuda.current_device():
        ws = _launch(p, q.device, dev)
    else:                              # the library plans and launches on the current device
        with torch.cuda.device(dev):
            ws = _launch(p, q.device, dev)
    # ws goes back to the caching allocator here; its reuse is ordered on this stream.
    del ws
    return out


def _launch(p: _lib.Params, device: torch.device, index: int):
    """Size and attach the split workspace, then launch on the current stream
    of ``device``. Returns the workspace tensor (or None) so the caller keeps
    it alive until the launch is enqueued."""
    ws = None
    ws_bytes = _lib.workspace_bytes(p)
    if ws_bytes:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
        p.workspace, p.workspace_bytes = ws.data_ptr(), ws_bytes
    _lib.fwd(p, torch._C._cuda_getCurrentRawStream(index))
    return ws


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


def num_splits_for(q, k, v, mask, variant=None) -> int:
    """The split count the library would use for these inputs (host query)."""
    validate(q, k, v, mask)
    p = make_params(q, k, v, mask, q, 0, variant)   # planning reads shapes only; q stands in for out
    with torch.cuda.device(q.device):
        return _lib.num_splits(p)
