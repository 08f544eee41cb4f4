"""Reference helpers shared by the GPU tests (torch fp32 reference on the device).

``ref_attn_torch`` restates the reference test's ground truth
(tests/test_mha_fwd_with_mask.py:38-53 of Defyli/custom_ops) per (b, h) so
full-size configs fit in memory: fp32 scores, amax.clamp_min(-1e30),
sum.clamp_min(1e-38), normalised P cast to the input dtype before P·V.
"""
import torch

ATOL = 2e-2
RTOL = 2e-2


def ref_attn_torch(q, k, v, mask, p_dtype=None):
    B, H, Sq, d = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    ratio = H // Hk
    scale = 1.0 / (d ** 0.5)
    p_dtype = p_dtype or v.dtype
    out = torch.empty(B, H, Sq, d, dtype=torch.float32, device=q.device)
    for b in range(B):
        mb = mask[b, 0, :Sq, :Sk].float()
        for h in range(H):
            s = (q[b, h].float() * scale) @ k[b, h // ratio].float().T + mb
            s = s - s.amax(dim=-1, keepdim=True).clamp_min(-1e30)
            e = torch.exp(s)
            p = (e / e.sum(dim=-1, keepdim=True).clamp_min(1e-38)).to(p_dtype)
            out[b, h] = p.float() @ v[b, h // ratio].float()
    return out


def assert_close(out, ref, name="", atol=ATOL, rtol=RTOL):
    o = out.float()
    r = ref.float()
    assert not torch.isnan(o).any(), f"{name}: NaN in output"
    err = (o - r).abs()
    bound = atol + rtol * r.abs()
    bad = err > bound
    if bad.any():
        idx = bad.nonzero()[0].tolist()
        raise AssertionError(f"{name}: {int(bad.sum())} elements out of tolerance; "
                             f"max_err={err.max().item():.3e} first at {idx}: "
                             f"out={o[tuple(idx)].item():.5f} ref={r[tuple(idx)].item():.5f}")
    return err.max().item()
