"""mi355_fa_fwd_noalloc (split partials, and for masks with unaligned rows the
live-tile map and the staged mask copy, in the library's per-GPU scratch array,
no workspace, no allocation) against mi355_fa_fwd with a caller workspace, both
called through the C-ABI: bit-identical outputs on two calls in a row (the
second smaller, so stale scratch contents from the first must not leak in), a
staged copy too large for the array replaced by the mask read in place, and a
clear rejection of a plan whose partials exceed the array.
"""
import ctypes

import pytest
import torch

from custom_ops_amd import _lib
from custom_ops_amd.fa import make_params

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20


def _inputs(b, h, hk, sq, sk, d, seed, dtype=torch.bfloat16):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(b, h, sq, d, generator=g, device="cuda").to(dtype)
    k = torch.randn(b, hk, sk, d, generator=g, device="cuda").to(dtype)
    v = torch.randn(b, hk, sk, d, generator=g, device="cuda").to(dtype)
    keep = torch.rand(b, 1, sq, sk, generator=g, device="cuda") > 0.1
    mask = torch.zeros(b, 1, sq, sk, device="cuda").masked_fill(~keep, float("-inf")).to(dtype)
    mask[..., :64] = 0
    return q, k, v, mask


def _run(entry, q, k, v, mask, splits, variant=None):
    lib = _lib.load()
    out = torch.full_like(q, float("nan"))
    p = make_params(q, k, v, mask, out, splits, variant)
    ws = None
    if entry == "fwd":
        n = lib.mi355_fa_workspace_bytes(ctypes.byref(p))
        if n:
            ws = torch.empty(n, dtype=torch.uint8, device="cuda")
            p.workspace, p.workspace_bytes = ws.data_ptr(), n
    else:
        # a workspace handed to the no-allocation entry point is ignored
        p.workspace, p.workspace_bytes = None, 0
    err = ctypes.create_string_buffer(512)
    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.mi355_fa_fwd if entry == "fwd" else lib.mi355_fa_fwd_noalloc
    rc = fn(ctypes.byref(p), stream, err, 512)
    assert rc == 0, err.value.decode()
    torch.cuda.synchronize()
    del ws
    return out, lib.mi355_fa_workspace_bytes(ctypes.byref(p))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_workspace_entry_two_calls(dtype):
    cases = [
        # (b, h, hk, sq, sk, d, splits): the first fills most of the array,
        # the second is smaller and reuses it
        (1, 16, 16, 128, 16384, 128, 16, 11),
        (1, 4, 2, 100, 3001, 64, 5, 12),
        # unsplit, unaligned mask rows: the staged mask (and no map: the
        # assembly loop does not narrow unsplit launches) in the array
        (2, 4, 4, 300, 777, 128, 1, 13),
    ]
    for b, h, hk, sq, sk, d, splits, seed in cases:
        q, k, v, mask = _inputs(b, h, hk, sq, sk, d, seed, dtype)
        ref, need = _run("fwd", q, k, v, mask, splits)
        got, _ = _run("noalloc", q, k, v, mask, splits)
        assert 0 < need <= SCRATCH, need
        assert not torch.isnan(ref).any()
        assert torch.equal(got, ref), (b, h, sq, sk, d, splits)


def test_noalloc_unsplit_needs_no_scratch():
    q, k, v, mask = _inputs(2, 4, 4, 300, 776, 128, 13)
    ref, need = _run("fwd", q, k, v, mask, 1)
    got, _ = _run("noalloc", q, k, v, mask, 1)
    assert need == 0
    assert torch.equal(got, ref)


def test_noalloc_reads_the_mask_in_place_when_the_copy_does_not_fit():
    """[4, 1, 2048, 2047] staged is 32 MiB plus its padding: beyond the array,
    so the no-allocation entry point plans without the copy, like
    mi355_fa_fwd with Variant(stage=-1)."""
    q, k, v, mask = _inputs(4, 2, 2, 2048, 2047, 128, 15)
    lib = _lib.load()
    p = make_params(q, k, v, mask, q, 1)
    assert lib.mi355_fa_workspace_bytes(ctypes.byref(p)) > SCRATCH
    ref, _ = _run("fwd", q, k, v, mask, 1, _lib.Variant(stage=-1))
    got, _ = _run("noalloc", q, k, v, mask, 1)
    assert not torch.isnan(ref).any()
    assert torch.equal(got, ref)
    staged, _ = _run("fwd", q, k, v, mask, 1)
    assert (staged.float() - ref.float()).abs().max().item() < 2e-2


def test_noalloc_rejects_plans_beyond_the_array():
    lib = _lib.load()
    q, k, v, mask = _inputs(4, 16, 16, 2048, 256, 128, 14)
    out = torch.zeros_like(q)
    p = make_params(q, k, v, mask, out, 4)   # 4 splits of 4·16·2048 rows: 128 MiB of partials
    assert lib.mi355_fa_workspace_bytes(ctypes.byref(p)) > SCRATCH
    err = ctypes.create_string_buffer(512)
    rc = lib.mi355_fa_fwd_noalloc(ctypes.byref(p), torch.cuda.current_stream().cuda_stream, err, 512)
    torch.cuda.synchronize()
    assert rc == _lib.EWORKSPACE
    assert "at most" in err.value.decode()
    assert torch.count_nonzero(out) == 0   # nothing was launched
