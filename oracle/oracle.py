"""CPU oracle for the masked FlashAttention forward (``mha_fwd_with_mask``).

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker / CPU baseline. The product package ``custom_ops_amd`` never imports it
and has no CPU fallback.

Three restatements of the reference's math, each pinned differently
(see tests/test_oracle.py):

* ``attn_fp64``      — closed form softmax(q·kᵀ·scale + mask)·v in float64 with
                       the reference's fully-masked-row convention (output 0).
* ``ref_attn_np``    — numpy mirror of the reference's test ground truth
                       ``ref_attn`` (tests/test_mha_fwd_with_mask.py:38-53):
                       fp32 scores, amax.clamp_min(-1e30), sum.clamp_min(1e-38),
                       normalised P cast to the input dtype before P·V.
* ``oracle_fwd``     — ctypes binding of ``fa_oracle.c``: the kernel's tile-wise
                       online softmax (csrc/fa/common/softmax.h:65-151), P rounded
                       to the dtype (csrc/fa/sm89/fa_fwd_kernel.h:384), optional
                       split-KV + LSE combine (fa_fwd_kernel.h:1406-1545).
* ``torch_math_cpu`` — the reference's CPU path as the benchmark defines it:
                       PyTorch fp32 math attention on host cores, chunked per
                       (b, h) to bound memory. Used as the timed CPU baseline.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile fa_oracle.c → oracle/liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH) or (
            os.path.getmtime(_LIB_PATH) < os.path.getmtime(os.path.join(_HERE, "fa_oracle.c"))):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        fp = ctypes.POINTER(ctypes.c_float)
        lib.oracle_mha_fwd.argtypes = [fp, fp, fp, fp, fp] + [ctypes.c_int] * 6 + [
            ctypes.c_int64, ctypes.c_int64, ctypes.c_float, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_int]
        lib.oracle_mha_fwd.restype = None
        lib.oracle_num_splits.argtypes = [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_float,
                                                                 ctypes.c_int]
        lib.oracle_num_splits.restype = ctypes.c_int
        lib.oracle_round.argtypes = [ctypes.c_float, ctypes.c_int]
        lib.oracle_round.restype = ctypes.c_float
        _lib = lib
    return _lib


# ── dtype helpers (bit-exact widening of 16-bit storage) ─────────────────────
ROUND_MODE = {"fp32": 0, "bf16": 1, "fp16": 2}


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 → bf16 bit pattern (inf/nan passed through)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    special = (u & 0x7F800000) == 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(special, u >> 16, r)
    return r.astype(np.uint16)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    if dtype == "fp16":
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
    return np.asarray(x, np.float32)


# ── closed forms ──────────────────────────────────────────────────────────────
def _expand_kv(k: np.ndarray, h: int) -> np.ndarray:
    hk = k.shape[1]
    return np.repeat(k, h // hk, axis=1) if hk != h else k


def attn_fp64(q, k, v, mask, scale=None):
    """float64 closed form. q [B,H,Sq,d]; k,v [B,Hk,Sk,d]; mask [B,1,>=Sq,>=Sk]
    (cropped to [:Sq,:Sk]). Fully masked rows → 0 (reference convention,
    csrc/fa/common/softmax.h:144)."""
    q = np.asarray(q, np.float64)
    B, H, Sq, d = q.shape
    Sk = k.shape[2]
    k = _expand_kv(np.asarray(k, np.float64), H)
    v = _expand_kv(np.asarray(v, np.float64), H)
    m = np.asarray(mask, np.float64)[:, :, :Sq, :Sk]
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * scale + m
    mx = s.max(axis=-1, keepdims=True) if Sk > 0 else np.full(s.shape[:-1] + (1,), -np.inf)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp(s - mx)
    den = e.sum(axis=-1, keepdims=True)
    p = np.where(den > 0, e / np.where(den > 0, den, 1.0), 0.0)
    return np.einsum("bhqk,bhkd->bhqd", p, v)


def ref_attn_np(q, k, v, mask, dtype="bf16"):
    """Mirror of the reference test's ref_attn (tests/test_mha_fwd_with_mask.py:38-53)
    in numpy fp32; P (normalised) cast to the input dtype before P·V."""
    q = np.asarray(q, np.float32)
    B, H, Sq, d = q.shape
    Sk = k.shape[2]
    k = _expand_kv(np.asarray(k, np.float32), H)
    v = _expand_kv(np.asarray(v, np.float32), H)
    scale = np.float32(1.0 / (d ** 0.5))
    s = np.matmul(q * scale, np.swapaxes(k, -1, -2)) + np.asarray(mask, np.float32)[:, :, :Sq, :Sk]
    s = s - np.maximum(s.max(axis=-1, keepdims=True), np.float32(-1e30))
    with np.errstate(over="ignore"):
        e = np.exp(s)
    den = np.maximum(e.sum(axis=-1, keepdims=True), np.float32(1e-38))
    p = round_to((e / den).astype(np.float32), dtype)
    return np.matmul(p, v)


# ── C oracle ──────────────────────────────────────────────────────────────────
def _fptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def oracle_fwd(q, k, v, mask, dtype="bf16", scale=None, block_n=64, num_splits=1,
               round_partials=True):
    """C restatement of the reference kernel math. Arrays are fp32 values of
    the (already dtype-exact) inputs; mask may be larger than (Sq, Sk)."""
    lib = _load()
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    mask = np.ascontiguousarray(mask, np.float32)
    B, H, Sq, d = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    out = np.zeros((B, H, Sq, d), np.float32)
    scale = float(1.0 / np.sqrt(d)) if scale is None else float(scale)
    mode = ROUND_MODE[dtype]
    mbs = mask.shape[1] * mask.shape[2] * mask.shape[3]
    mrs = mask.shape[3]
    lib.oracle_mha_fwd(_fptr(q), _fptr(k), _fptr(v), _fptr(mask), _fptr(out), B, H, Hk, Sq, Sk,
                       d, mbs, mrs, scale, mode, block_n, num_splits,
                       mode if round_partials else 0)
    return out


def oracle_num_splits(total_mblocks, num_n_blocks, block_m, head_dim, num_sms, K, P0=0.35,
                      max_splits=64):
    return _load().oracle_num_splits(total_mblocks, num_n_blocks, block_m, head_dim, num_sms,
                                     K, P0, max_splits)


def oracle_round_scalar(x: float, dtype: str) -> float:
    return _load().oracle_round(x, ROUND_MODE[dtype])


# ── PyTorch CPU math path (the reported CPU baseline) ─────────────────────────
def torch_math_cpu(q, k, v, mask, heads=None):
    """PyTorch fp32 math attention on host cores, the reference's "CPU path"
    (same formula as tests/test_mha_fwd_with_mask.py:38-53, P kept in fp32).
    Processes one (b, h) at a time; ``heads`` restricts to a list of (b, h).
    The per-head score, max, sum and output buffers are allocated once per call
    and reused (in-place ops), so the timing measures the math rather than
    the host allocator's page faults."""
    import torch
    B, H, Sq, d = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    ratio = H // Hk
    scale = 1.0 / (d ** 0.5)
    out = torch.zeros(B, H, Sq, d, dtype=torch.float32)
    todo = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    s = torch.empty(Sq, Sk, dtype=torch.float32)
    mx = torch.empty(Sq, 1, dtype=torch.float32)
    sm = torch.empty(Sq, 1, dtype=torch.float32)
    qs = torch.empty(Sq, d, dtype=torch.float32)
    for b, h in todo:
        torch.mul(q[b, h].float(), scale, out=qs)
        kf = k[b, h // ratio].float()
        vf = v[b, h // ratio].float()
        torch.matmul(qs, kf.T, out=s)
        s.add_(mask[b, 0, :Sq, :Sk].float())
        torch.amax(s, dim=-1, keepdim=True, out=mx)
        s.sub_(mx.clamp_min_(-1e30))
        s.exp_()
        torch.sum(s, dim=-1, keepdim=True, out=sm)
        s.div_(sm.clamp_min_(1e-38))
        torch.matmul(s, vf, out=out[b, h])
    return out
