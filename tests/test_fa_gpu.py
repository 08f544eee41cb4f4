"""GPU parity tests for recsys_ops::mha_fwd_with_mask on MI355X.

Case matrix follows the reference's own tests (Defyli/custom_ops):
tests/test_mha_fwd_with_mask.py:181-230 (base, mask kinds, unaligned, tails,
Sq=1, pre-padded masks with trap values, split-KV, GQA, error paths) and
tests/remote_verify_suite.py:108-161 (ragged Sk/Sq sweeps, GQA ratios, mask
pre-pad with unaligned widths, long split-KV, finite bias masks).

Ground truth: the torch fp32 restatement of the reference's ref_attn (tests/_ref.py)
for every case, and the C oracle (oracle/fa_oracle.c) on small cases.
Tolerance (north_star): |out − ref| ≤ 2e-2 + 2e-2·|ref| elementwise, no NaN;
fully-masked rows must be exactly 0.
"""
import numpy as np
import pytest
import torch

from tests._ref import ATOL, RTOL, assert_close, ref_attn_torch

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16]


@pytest.fixture(scope="module")
def ops(gpu):
    from custom_ops_amd import ops as _ops
    _ops.ensure_loaded()
    return _ops


def _rand(shape, g, scale=0.5):
    return torch.randn(*shape, generator=g) * scale


def make_case(b, h, hk, sq, sk, d, kind, dtype, seed=42, extra_rows=0, extra_cols=0):
    g = torch.Generator().manual_seed(seed)
    q = _rand((b, h, sq, d), g).to(dtype)
    k = _rand((b, hk, sk, d), g).to(dtype)
    v = _rand((b, hk, sk, d), g).to(dtype)
    sqm, skm = sq + extra_rows, sk + extra_cols
    if kind == "zero":
        m = torch.zeros(b, 1, sqm, skm)
    elif kind == "causal":
        m = torch.triu(torch.full((sqm, skm), float("-inf")), diagonal=1).expand(b, 1, sqm, skm)
    elif kind == "random":        # finite N(0, 0.3) bias (reference "random")
        m = torch.randn(b, 1, sqm, skm, generator=g) * 0.3
    elif kind == "block":
        m = torch.zeros(b, 1, sqm, skm)
        m[..., sk // 2:] = float("-inf")
    elif kind == "all_masked_row":
        m = torch.zeros(b, 1, sqm, skm)
        m[:, :, 0, :] = float("-inf")
    elif kind == "inf_random":    # ~1/7 i.i.d. -inf (remote_verify_suite "random")
        m = torch.zeros(b, 1, sqm, skm).masked_fill(
            torch.rand(b, 1, sqm, skm, generator=g) < 1.0 / 7.0, float("-inf"))
    elif kind == "bias":          # ALiBi-like finite bias
        pos = torch.arange(skm, dtype=torch.float32)
        m = ((pos % 16) - 8).view(1, 1, 1, -1).expand(b, 1, sqm, skm)
    elif kind == "full_row":
        m = torch.zeros(b, 1, sqm, skm)
        m[:, :, sqm // 3, :] = float("-inf")
    else:
        raise ValueError(kind)
    if extra_cols:   # trap values in the pad columns: visible-looking numbers
        m = m.clone()
        m[..., sk:] = torch.randn(b, 1, sqm, extra_cols, generator=g) * 0.3
    return q, k, v, m.contiguous().to(dtype)


def run(ops, case, dev, name, num_splits=0, waves=0):
    q, k, v, m = (t.to(dev) for t in case)
    if num_splits or waves:
        from custom_ops_amd import Variant, mha_fwd_with_mask
        out = mha_fwd_with_mask(q, k, v, m, num_splits=num_splits, variant=Variant(waves=waves))
    else:
        out = ops.mha_fwd_with_mask(q, k, v, m)
    torch.cuda.synchronize()
    assert out.dtype == q.dtype and out.shape == q.shape
    ref = ref_attn_torch(q, k, v, m)
    assert_close(out, ref, name)
    return out, ref


# ── base paths and mask semantics (test_mha_fwd_with_mask.py:184-195) ────────
BASE = [(2, 16, 256, 256, 64), (2, 16, 256, 256, 128), (1, 24, 512, 384, 64),
        (1, 24, 384, 512, 128)]


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16"])
@pytest.mark.parametrize("shape", BASE, ids=lambda s: "x".join(map(str, s)))
def test_base_zero_mask(ops, gpu, dtype, shape):
    b, h, sq, sk, d = shape
    run(ops, make_case(b, h, h, sq, sk, d, "zero", dtype), gpu, f"base{shape}")


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16"])
@pytest.mark.parametrize("kind", ["causal", "random", "block", "all_masked_row", "inf_random",
                                  "bias"])
@pytest.mark.parametrize("d", [64, 128])
def test_mask_kinds(ops, gpu, dtype, kind, d):
    out, _ = run(ops, make_case(2, 16, 16, 256, 256, d, kind, dtype), gpu, f"{kind}_d{d}")
    if kind == "all_masked_row":
        assert torch.all(out[:, :, 0, :] == 0), "fully-masked row must be exactly 0"


# ── unaligned shapes, tails, Sq=1 (test_mha_fwd_with_mask.py:197-214) ─────────
UNALIGNED = [
    (1, 8, 100, 104, 64, "zero"), (1, 8, 100, 200, 128, "random"),
    (1, 8, 256, 1032, 128, "random"), (1, 8, 64, 56, 64, "random"),
    (1, 8, 128, 8, 128, "causal"), (1, 4, 1, 104, 64, "random"),
    (1, 2, 128, 1032, 128, "random"),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", UNALIGNED, ids=lambda c: "x".join(map(str, c)))
def test_unaligned(ops, gpu, dtype, case):
    b, h, sq, sk, d, kind = case
    run(ops, make_case(b, h, h, sq, sk, d, kind, dtype), gpu, f"unaligned{case}")


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16"])
@pytest.mark.parametrize("rows,cols", [(0, 8), (8, 8), (13, 5), (0, 3)])
def test_mask_prepadded_traps(ops, gpu, dtype, rows, cols):
    """Mask larger than (Sq, Sk) with visible-looking trap values in the pad:
    they must be ignored (col >= Sk always blocked; rows >= Sq dropped)."""
    q, k, v, m = (t.to(gpu) for t in make_case(1, 8, 8, 100, 104, 64, "random", dtype,
                                               extra_rows=rows, extra_cols=cols))
    from custom_ops_amd import ops as o
    out = o.mha_fwd_with_mask(q, k, v, m)
    ref = ref_attn_torch(q, k, v, m[:, :, :100, :104].contiguous())
    assert_close(out, ref, f"prepad+{rows}r+{cols}c")


# ── ragged sweeps (remote_verify_suite.py:108-161) ─────────────────────────────
@pytest.mark.parametrize("sk", [1, 7, 9, 55, 63, 100, 101, 777, 1031, 2053, 4099])
def test_ragged_sk(ops, gpu, sk):
    run(ops, make_case(1, 4, 2, 64, sk, 128, "inf_random", torch.bfloat16), gpu, f"sk{sk}")


@pytest.mark.parametrize("sq", [1, 3, 63, 65, 127, 129, 333, 1000])
def test_ragged_sq(ops, gpu, sq):
    run(ops, make_case(1, 4, 4, sq, 256, 64, "inf_random", torch.bfloat16), gpu, f"sq{sq}")


@pytest.mark.parametrize("h,hk", [(2, 1), (8, 2), (12, 3), (16, 4), (32, 8)])
@pytest.mark.parametrize("d", [64, 128])
def test_gqa_vs_repeat_interleave(ops, gpu, h, hk, d):
    q, k, v, m = (t.to(gpu) for t in make_case(1, h, hk, 256, 384, d, "inf_random",
                                               torch.bfloat16))
    out = ops.mha_fwd_with_mask(q, k, v, m)
    r = h // hk
    out_mha = ops.mha_fwd_with_mask(q, k.repeat_interleave(r, 1).contiguous(),
                                    v.repeat_interleave(r, 1).contiguous(), m)
    torch.cuda.synchronize()
    assert torch.equal(out, out_mha), "GQA must equal MHA on repeat_interleaved K/V exactly"
    assert_close(out, ref_attn_torch(q, k, v, m), f"gqa{h}/{hk}")


# ── split-KV (test_mha_fwd_with_mask.py:216-224; remote suite :150-155) ────────
SPLIT = [(1, 1, 128, 8192, 64, "zero"), (1, 1, 64, 4096, 64, "causal"),
         (1, 40, 256, 4096, 64, "zero"), (1, 2, 128, 8192, 128, "zero"),
         (1, 2, 256, 16384, 128, "random"), (1, 2, 100, 8195, 128, "inf_random"),
         (1, 2, 64, 32773, 128, "inf_random")]


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", SPLIT, ids=lambda c: "x".join(map(str, c)))
def test_splitkv_auto(ops, gpu, dtype, case):
    b, h, sq, sk, d, kind = case
    run(ops, make_case(b, h, h, sq, sk, d, kind, dtype), gpu, f"split{case}")


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 16, 64])
def test_split_invariance(ops, gpu, splits):
    """Any forced split count gives the same answer (s = 1 is the base kernel)."""
    case = make_case(1, 4, 2, 96, 3000, 128, "inf_random", torch.bfloat16)
    case[3][:, :, 5, :] = float("-inf")   # one fully masked row
    out, _ = run(ops, case, gpu, f"splits={splits}", num_splits=splits)
    assert torch.all(out[:, :, 5, :] == 0)


@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16"])
@pytest.mark.parametrize("sk,extra_cols", [(1000, 0), (777, 3)])
def test_workgroup_variants(ops, gpu, waves, splits, d, dtype, sk, extra_cols):
    """Both workgroup sizes (4 waves / BM 128, 8 waves / BM 256), forced through
    the single-pass and split-KV epilogues, with 16-byte-aligned mask rows (LDS
    DMA) and unaligned ones (register path)."""
    case = make_case(2, 4, 2, 300, sk, d, "inf_random", dtype, extra_cols=extra_cols)
    case[3][1, :, 17, :] = float("-inf")
    out, _ = run(ops, case, gpu, f"w{waves} s{splits} d{d} sk{sk}", num_splits=splits, waves=waves)
    assert torch.all(out[1, :, 17, :] == 0)


def _skip_mask(kind, b, sq, sk, g):
    m = torch.zeros(b, 1, sq, sk)
    rows = torch.arange(sq).view(-1, 1)
    cols = torch.arange(sk).view(1, -1)
    if kind == "causal":              # bottom-right aligned causal
        m.masked_fill_(cols > rows + (sk - sq), float("-inf"))
    elif kind == "window":            # 256-key sliding window, bottom-right aligned
        off = rows + (sk - sq)
        m.masked_fill_((cols > off) | (cols < off - 255), float("-inf"))
    elif kind == "dead_stripes":      # whole 64-key tiles dead, then a lone live key
        dead = ((cols // 64) % 3 == 1) | ((cols // 64) % 5 == 2)
        m.masked_fill_(dead, float("-inf"))
        m[..., 64 * 4 + 17] = 0.0     # tile 4 is live again through one column
    elif kind == "pad_rows_cols":     # batch-1 keys >= sk-300 blocked, rows >= 400 see nothing
        m[1, :, :, sk - 300:] = float("-inf")
        m[:, :, 400:, :] = float("-inf")
    m.masked_fill_(torch.rand(b, 1, sq, sk, generator=g) < 0.05, float("-inf"))
    return m


@pytest.mark.parametrize("kind", ["causal", "window", "dead_stripes", "pad_rows_cols"])
@pytest.mark.parametrize("waves", [4, 8])
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float16, 64)],
                         ids=["bf16d128", "fp16d64"])
def test_dead_mask_blocks(ops, gpu, kind, waves, splits, dtype, d):
    """Masks with whole 32-row x 64-key blocks at -inf (a wave skips the
    softmax / PV work of a tile in which none of its rows sees a key): results
    match the fp32 reference, and rows that see no key are exactly 0."""
    from custom_ops_amd import Variant, mha_fwd_with_mask
    g = torch.Generator().manual_seed(7)
    b, h, hk, sq, sk = 2, 4, 2, 700, 1500
    q = _rand((b, h, sq, d), g).to(dtype).to(gpu)
    k = _rand((b, hk, sk, d), g).to(dtype).to(gpu)
    v = _rand((b, hk, sk, d), g).to(dtype).to(gpu)
    m = _skip_mask(kind, b, sq, sk, g).to(dtype).to(gpu)
    out = mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=Variant(waves=waves))
    torch.cuda.synchronize()
    assert_close(out, ref_attn_torch(q, k, v, m), f"dead blocks {kind} w{waves} s{splits} d{d}")
    dead_rows = torch.isinf(m).all(-1).squeeze(1)          # [b, sq]
    assert torch.all(out.permute(0, 2, 1, 3)[dead_rows] == 0)


def _sweep_cases(n=48, seed=2024):
    """Seeded random shapes over the op's whole contract."""
    import random
    rnd = random.Random(seed)
    kinds = ["zero", "causal", "random", "block", "all_masked_row", "inf_random", "bias",
             "full_row"]
    cases = []
    for i in range(n):
        d = rnd.choice([64, 128])
        hk = rnd.choice([1, 2, 4])
        h = hk * rnd.choice([1, 2, 4])
        b = rnd.choice([1, 2, 3])
        sq = rnd.choice([1, 2, 17, 64, 100, 129, 255, 256, 257, 400, 513])
        sk = rnd.choice([1, 5, 8, 31, 64, 65, 127, 200, 511, 777, 1024, 1500, 3001])
        dtype = rnd.choice(["bf16", "fp16"])
        kind = rnd.choice(kinds)
        pad_r, pad_c = rnd.choice([(0, 0), (0, 0), (3, 0), (0, 5), (7, 8)])
        splits = rnd.choice([0, 0, 0, 1, 2, 5])
        cases.append((i, b, h, hk, sq, sk, d, dtype, kind, pad_r, pad_c, splits))
    return cases


@pytest.mark.parametrize("case", _sweep_cases(), ids=lambda c: f"sweep{c[0]}")
def test_random_shape_sweep(ops, gpu, case):
    """Randomised (seeded) coverage of the contract: MHA and GQA, d 64/128,
    bf16/fp16, ragged Sq/Sk, pre-padded masks with trap values, every mask
    kind, automatic and forced split counts."""
    i, b, h, hk, sq, sk, d, dtype, kind, pad_r, pad_c, splits = case
    dt = torch.bfloat16 if dtype == "bf16" else torch.float16
    c = make_case(b, h, hk, sq, sk, d, kind, dt, seed=1000 + i, extra_rows=pad_r,
                  extra_cols=pad_c)
    out, _ = run(ops, c, gpu, f"sweep{i} {case[1:]}", num_splits=splits)
    rows_dead = torch.isinf(c[3][:, 0, :sq, :sk].float()).all(-1)       # [b, sq]
    assert torch.all(out.permute(0, 2, 1, 3)[rows_dead.to(gpu)] == 0)



def _sweep_cases_large(n=24, seed=77):
    """Larger seeded shapes: several 256-row blocks (both tile orders), long Sk
    with automatic splits, GQA up to 8:1, forced workgroup sizes."""
    import random
    rnd = random.Random(seed)
    kinds = ["zero", "causal", "random", "inf_random", "bias", "full_row", "block"]
    cases = []
    while len(cases) < n:
        d = rnd.choice([64, 128])
        hk = rnd.choice([1, 2, 4, 8])
        h = hk * rnd.choice([1, 2, 4, 8])
        b = rnd.choice([1, 2])
        sq = rnd.choice([300, 511, 700, 1024, 1100])
        sk = rnd.choice([2049, 4096, 5000, 9001])
        if b * h * sq * sk > 5e7:
            continue
        cases.append((len(cases), b, h, hk, sq, sk, d, rnd.choice(["bf16", "fp16"]),
                      rnd.choice(kinds), rnd.choice([(0, 0), (0, 0), (5, 3)]),
                      rnd.choice([0, 0, 0, 3]), rnd.choice([0, 0, 4, 8])))
    return cases


@pytest.mark.parametrize("case", _sweep_cases_large(), ids=lambda c: f"large{c[0]}")
def test_random_shape_sweep_large(ops, gpu, case):
    i, b, h, hk, sq, sk, d, dtype, kind, (pad_r, pad_c), splits, waves = case
    dt = torch.bfloat16 if dtype == "bf16" else torch.float16
    c = make_case(b, h, hk, sq, sk, d, kind, dt, seed=5000 + i, extra_rows=pad_r,
                  extra_cols=pad_c)
    out, _ = run(ops, c, gpu, f"large{i} {case[1:]}", num_splits=splits, waves=waves)
    rows_dead = torch.isinf(c[3][:, 0, :sq, :sk].float()).all(-1)
    assert torch.all(out.permute(0, 2, 1, 3)[rows_dead.to(gpu)] == 0)


def test_all_masked_everything_split(ops, gpu):
    q, k, v, m = make_case(1, 2, 2, 64, 4096, 128, "zero", torch.bfloat16)
    m = torch.full_like(m, float("-inf"))
    from custom_ops_amd import mha_fwd_with_mask
    for s in (1, 4):
        out = mha_fwd_with_mask(q.to(gpu), k.to(gpu), v.to(gpu), m.to(gpu), num_splits=s)
        torch.cuda.synchronize()
        assert torch.all(out == 0) and not torch.isnan(out).any()


# ── error paths (test_mha_fwd_with_mask.py:131-170) ────────────────────────────
def test_error_paths(ops, gpu):
    # Sk % 8 != 0 → handled (auto-pad semantics), result correct
    g = torch.Generator().manual_seed(1)
    q = torch.randn(1, 1, 64, 64, generator=g).half().to(gpu)
    k = torch.randn(1, 1, 100, 64, generator=g).half().to(gpu)
    v = torch.randn(1, 1, 100, 64, generator=g).half().to(gpu)
    m = torch.zeros(1, 1, 64, 100, dtype=torch.float16, device=gpu)
    m[..., ::7] = float("-inf")
    assert_close(ops.mha_fwd_with_mask(q, k, v, m), ref_attn_torch(q, k, v, m), "autopad")
    # fp32 input raises
    qf = torch.randn(1, 1, 64, 64, device=gpu)
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        ops.mha_fwd_with_mask(qf, qf, qf, torch.zeros(1, 1, 64, 64, device=gpu))
    # mixed dtypes raise
    kb = torch.randn(1, 1, 64, 64, device=gpu).bfloat16()
    with pytest.raises(RuntimeError, match="k dtype must match q"):
        ops.mha_fwd_with_mask(q, kb, q, torch.zeros(1, 1, 64, 64, dtype=torch.float16,
                                                    device=gpu))
    with pytest.raises(RuntimeError, match="head_dim"):
        x = torch.zeros(1, 1, 8, 96, dtype=torch.float16, device=gpu)
        ops.mha_fwd_with_mask(x, x, x, torch.zeros(1, 1, 8, 8, dtype=torch.float16, device=gpu))
    with pytest.raises(RuntimeError, match="divisible"):
        a = torch.zeros(1, 3, 8, 64, dtype=torch.float16, device=gpu)
        bb = torch.zeros(1, 2, 8, 64, dtype=torch.float16, device=gpu)
        ops.mha_fwd_with_mask(a, bb, bb, torch.zeros(1, 1, 8, 8, dtype=torch.float16,
                                                     device=gpu))
    with pytest.raises(RuntimeError, match="mask shape"):
        a = torch.zeros(1, 2, 8, 64, dtype=torch.float16, device=gpu)
        ops.mha_fwd_with_mask(a, a, a, torch.zeros(1, 1, 7, 8, dtype=torch.float16,
                                                   device=gpu))
    with pytest.raises(RuntimeError, match="contiguous"):
        a = torch.zeros(1, 2, 64, 8, dtype=torch.float16, device=gpu).transpose(2, 3)
        ops.mha_fwd_with_mask(a, a, a, torch.zeros(1, 1, 8, 8, dtype=torch.float16,
                                                   device=gpu))


def test_autopad_equals_explicit_pad(ops, gpu):
    """Sk % 8 != 0 must equal the reference's explicit pad (K/V zero rows, mask
    -inf columns; csrc/fa/fa_fwd_op.cu:117-134) — bit for bit."""
    q, k, v, m = (t.to(gpu) for t in make_case(2, 4, 2, 130, 1001, 128, "inf_random",
                                               torch.bfloat16))
    out = ops.mha_fwd_with_mask(q, k, v, m)
    pad = 1008 - 1001
    kp = torch.nn.functional.pad(k, (0, 0, 0, pad))
    vp = torch.nn.functional.pad(v, (0, 0, 0, pad))
    mp = torch.nn.functional.pad(m, (0, pad), value=float("-inf"))
    out_p = ops.mha_fwd_with_mask(q, kp.contiguous(), vp.contiguous(), mp.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(out, out_p)


def test_empty_and_sk0(ops, gpu):
    z = torch.zeros(0, 2, 8, 64, dtype=torch.bfloat16, device=gpu)
    out = ops.mha_fwd_with_mask(z, z, z, torch.zeros(0, 1, 8, 8, dtype=torch.bfloat16,
                                                     device=gpu))
    assert out.shape == z.shape
    q = torch.randn(1, 2, 8, 64, device=gpu).bfloat16()
    k = torch.zeros(1, 2, 0, 64, dtype=torch.bfloat16, device=gpu)
    out = ops.mha_fwd_with_mask(q, k, k, torch.zeros(1, 1, 8, 0, dtype=torch.bfloat16,
                                                     device=gpu))
    torch.cuda.synchronize()
    assert torch.all(out == 0)


# ── C oracle and committed fixtures ────────────────────────────────────────────
def test_vs_c_oracle_small(ops, gpu):
    from oracle import oracle as orc
    for dtype, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        q, k, v, m = make_case(2, 4, 2, 72, 133, 64, "inf_random", dtype, seed=7)
        m[:, :, 3, :] = float("-inf")
        out = ops.mha_fwd_with_mask(q.to(gpu), k.to(gpu), v.to(gpu), m.to(gpu)).cpu()
        ref = orc.oracle_fwd(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                             m.float().numpy(), dtype=name)
        assert_close(out, torch.from_numpy(ref), f"oracle-{name}")
        assert torch.all(out[:, :, 3] == 0)



@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bf16"), (torch.float16, "fp16")])
@pytest.mark.parametrize("splits", [1, 3])
def test_finfo_min_masks(ops, gpu, dtype, name, splits):
    """Masks built the Hugging Face way, with torch.finfo(dtype).min as
    "blocked". The reference kernel adds mask·(1/scale) to the unscaled scores
    in fp32 (csrc/fa/sm89/fa_fwd_kernel.h:286-310): for bf16 that overflows to
    -inf, so a row of minima is fully masked and exactly 0; for fp16 it stays
    finite, so a row of minima is an ordinary softmax over q·k. The C oracle
    restates that arithmetic."""
    from custom_ops_amd import mha_fwd_with_mask
    from oracle import oracle as orc
    q, k, v, _ = make_case(2, 4, 2, 80, 200, 128, "zero", dtype, seed=11)
    g = torch.Generator().manual_seed(5)
    lo = torch.finfo(dtype).min
    m = torch.zeros(2, 1, 80, 200).masked_fill(torch.rand(2, 1, 80, 200, generator=g) < 0.3, lo)
    m[:, :, 5, :] = lo
    m[:, :, 6, :] = float("-inf")
    m = m.to(dtype)
    out = mha_fwd_with_mask(q.to(gpu), k.to(gpu), v.to(gpu), m.to(gpu), num_splits=splits).cpu()
    ref = torch.from_numpy(orc.oracle_fwd(q.float().numpy(), k.float().numpy(),
                                          v.float().numpy(), m.float().numpy(), dtype=name))
    assert_close(out, ref, f"finfo-min-{name}-s{splits}")
    assert torch.all(out[:, :, 6] == 0)
    if dtype == torch.bfloat16:
        assert torch.all(out[:, :, 5] == 0)
    else:
        assert torch.all(torch.isfinite(out[:, :, 5].float())) and out[:, :, 5].abs().sum() > 0



@pytest.mark.parametrize("slope", [0.2, -0.2, 0.02])
@pytest.mark.parametrize("splits", [1, 4])
def test_moving_running_max(ops, gpu, slope, splits):
    """A mask bias that rises along the keys moves the running max on every
    64-key tile (0.2 per key = 12.8 per tile, past the lazy-rescale slack each
    time), a falling one never moves it after the first tile, a gentle one
    moves it every few tiles; logits reach about +-200."""
    from custom_ops_amd import mha_fwd_with_mask
    for dtype in (torch.bfloat16, torch.float16):
        q, k, v, _ = make_case(1, 2, 2, 64, 1024, 128, "zero", dtype, seed=3)
        ramp = (torch.arange(1024, dtype=torch.float32) * slope).view(1, 1, 1, -1)
        m = ramp.expand(1, 1, 64, 1024).contiguous().to(dtype)
        out = mha_fwd_with_mask(q.to(gpu), k.to(gpu), v.to(gpu), m.to(gpu), num_splits=splits)
        ref = ref_attn_torch(q.to(gpu), k.to(gpu), v.to(gpu), m.to(gpu))
        assert_close(out, ref, f"ramp{slope}-s{splits}-{dtype}")



@pytest.mark.parametrize("shape,splits", [((1, 4, 2, 200, 3000, 128), 0),   # auto: split
                                          ((2, 4, 4, 300, 700, 64), 1),    # unsplit
                                          ((1, 4, 2, 200, 3001, 128), 2),  # compiled kernel, fused tail
                                          ((1, 4, 2, 200, 3001, 128), 5),  # compiled kernel, combine
                                          ((2, 4, 4, 300, 777, 128), 1)])  # unsplit, live-tile map
def test_graph_capture_replays(ops, gpu, shape, splits):
    """The op captured in a HIP graph (workspace from the graph-aware caching
    allocator, no memset nodes) and replayed several times with new inputs
    copied into the captured buffers, eager work and synchronisations in
    between: every replay equals the eager result bit for bit. A replay reuses
    the captured launch tag and its own workspace, so the fused tail's ticket
    words count on across replays; masks with unaligned rows replay the
    live-tile map kernel before the attention kernel."""
    from custom_ops_amd import mha_fwd_with_mask
    b, h, hk, sq, sk, d = shape
    q, k, v, m = (t.to(gpu) for t in make_case(b, h, hk, sq, sk, d, "inf_random",
                                              torch.bfloat16, seed=21))
    fn = lambda: mha_fwd_with_mask(q, k, v, m, num_splits=splits)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    for seed in (1, 2, 3):
        nq, nk, nv, nm = (t.to(gpu) for t in make_case(b, h, hk, sq, sk, d, "inf_random",
                                                      torch.bfloat16, seed=seed))
        q.copy_(nq); k.copy_(nk); v.copy_(nv); m.copy_(nm)
        graph.replay()
        torch.cuda.synchronize()
        ref = fn()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay with seed {seed}"


def test_golden_fixtures(ops, gpu):
    from tests.golden import load_fixtures
    for fx in load_fixtures():
        q, k, v, m = (t.to(gpu) for t in fx.tensors_torch())
        out = ops.mha_fwd_with_mask(q, k, v, m).float().cpu().numpy()
        exp = fx.expected
        err = np.abs(out - exp)
        assert np.all(err <= ATOL + RTOL * np.abs(exp)), f"{fx.name}: max_err {err.max():.3e}"
        for r in fx.masked_rows:
            assert np.all(out[:, :, r, :] == 0), f"{fx.name}: masked row {r} not 0"


# ── benchmark configurations cfg2-cfg5 at full size ───────────────────────────────────────
@pytest.mark.parametrize("name", ["cfg2", "cfg3", "cfg4", "cfg5"])
def test_baseline_config(ops, gpu, name):
    from custom_ops_amd.workloads import CONFIGS, make_inputs
    cfg = CONFIGS[name]
    q, k, v, m = (t.to(gpu) for t in make_inputs(cfg))
    out = ops.mha_fwd_with_mask(q, k, v, m)
    torch.cuda.synchronize()
    ref = ref_attn_torch(q, k, v, m)
    assert_close(out, ref, name)


def test_baseline_cfg1_plumbing(ops, gpu):
    """cfg1 (fp32 causal, CPU plumbing) run through the bf16 device path vs the
    C oracle on the same bf16-rounded inputs."""
    from custom_ops_amd.workloads import CONFIGS, make_inputs
    from oracle import oracle as orc
    cfg = CONFIGS["cfg1"]
    q, k, v, m = (t.bfloat16() for t in make_inputs(cfg))
    out = ops.mha_fwd_with_mask(q.to(gpu), k.to(gpu), v.to(gpu), m.to(gpu)).float().cpu()
    ref = orc.oracle_fwd(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                         m.float().numpy(), dtype="bf16")
    assert_close(out, torch.from_numpy(ref), "cfg1")


def test_gqa_full_cfg3_equals_mha(ops, gpu):
    from custom_ops_amd.workloads import CONFIGS, make_inputs
    q, k, v, m = (t.to(gpu) for t in make_inputs(CONFIGS["cfg3"]))
    out = ops.mha_fwd_with_mask(q, k, v, m)
    out2 = ops.mha_fwd_with_mask(q, k.repeat_interleave(4, 1).contiguous(),
                                 v.repeat_interleave(4, 1).contiguous(), m)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_shift_invariance_cfg5(ops, gpu):
    """Adding a constant to every mask entry of a row leaves softmax unchanged."""
    from custom_ops_amd.workloads import CONFIGS, make_inputs
    q, k, v, m = (t.to(gpu) for t in make_inputs(CONFIGS["cfg5"]))
    out = ops.mha_fwd_with_mask(q, k, v, m)
    out2 = ops.mha_fwd_with_mask(q, k, v, (m.float() + 2.0).to(m.dtype))
    torch.cuda.synchronize()
    assert_close(out2, out.float(), "shift", atol=1e-2, rtol=1e-2)


def test_stream_semantics(ops, gpu):
    """Work is enqueued on the caller's current stream (no implicit sync)."""
    q, k, v, m = (t.to(gpu) for t in make_case(1, 4, 4, 256, 512, 128, "inf_random",
                                               torch.bfloat16))
    ref = ops.mha_fwd_with_mask(q, k, v, m)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = ops.mha_fwd_with_mask(q, k, v, m)
    s.synchronize()
    assert torch.equal(out, ref)


def test_random_fuzz_vs_reference(ops, gpu):
    """300 seeded random cases through the op with the library's own plan:
    B 1-3, GQA ratios 1-8, Sq 1-2500, Sk 1-9000, d 64/128, bf16/fp16, mask
    rows/columns beyond Sq/Sk (pad columns hold visible-looking trap values),
    and random / causal / finite-bias / sliding-window / masked-row masks.
    Every output within the fp32 reference's tolerance, no NaN, rows with no
    visible key exactly 0."""
    import random
    from custom_ops_amd import mha_fwd_with_mask
    rng = random.Random(7)
    for i in range(300):
        b = rng.choice([1, 1, 2, 3]); hk = rng.choice([1, 2, 4]); h = hk * rng.choice([1, 2, 4, 8])
        sq = rng.choice([1, 7, 64, 100, 128, 255, 257, 600, 1000, 2048, 2500])
        sk = rng.choice([1, 9, 63, 64, 65, 500, 1024, 1500, 4099, 9000])
        if b * h * sq * sk > 6e7:
            sk = max(1, int(6e7 // (b * h * sq)))
        d = rng.choice([64, 128]); dt = rng.choice([torch.bfloat16, torch.float16])
        er = rng.choice([0, 0, 3]); ec = rng.choice([0, 0, 5, 8])
        kind = rng.choice(["rand", "causal", "bias", "window", "rows"])
        g = torch.Generator(device=gpu).manual_seed(1000 + i)
        q = (torch.randn(b, h, sq, d, generator=g, device=gpu) * 0.6).to(dt)
        k = (torch.randn(b, hk, sk, d, generator=g, device=gpu) * 0.6).to(dt)
        v = (torch.randn(b, hk, sk, d, generator=g, device=gpu) * 0.6).to(dt)
        m = torch.zeros(b, 1, sq + er, sk + ec, device=gpu)
        r = torch.arange(sq + er, device=gpu).view(-1, 1)
        c = torch.arange(sk + ec, device=gpu).view(1, -1)
        if kind == "rand":
            m.masked_fill_(torch.rand(m.shape, generator=g, device=gpu) < 0.2, float("-inf"))
        elif kind == "causal":
            m.masked_fill_(c > r + (sk - sq), float("-inf"))
        elif kind == "bias":
            m += torch.randn(m.shape, generator=g, device=gpu) * 2.0
        elif kind == "window":
            off = r + (sk - sq)
            m.masked_fill_((c > off) | (c <= off - 300), float("-inf"))
        else:
            m[:, :, ::7, :] = float("-inf")
        if ec:
            m[..., sk:] = 1.0
        m = m.to(dt)
        case = dict(i=i, b=b, h=h, hk=hk, sq=sq, sk=sk, d=d, dtype=str(dt), kind=kind, er=er, ec=ec)
        out = mha_fwd_with_mask(q, k, v, m)
        assert_close(out, ref_attn_torch(q, k, v, m), str(case))
        dead = torch.isinf(m[:, :, :sq, :sk].float()).all(-1).squeeze(1)   # [b, sq]
        if dead.any():
            assert torch.all(out.permute(0, 2, 1, 3)[dead] == 0), str(case)


def test_random_fuzz_variants_vs_reference(ops, gpu):
    """300 seeded random cases as above, each with a random kernel variant and
    split count: the staged mask copy forced on or off, the live-tile map
    forced on or off, live-range narrowing forced on, the compiled kernel, 4-
    or 8-wave workgroups, 2-7 splits; plus key-padding masks (a dead tail of
    random length per batch) and masks with periodic dead tile runs. Every
    output within the fp32 reference's tolerance, rows with no visible key
    exactly 0."""
    import random
    from custom_ops_amd import Variant, mha_fwd_with_mask
    rng = random.Random(11)
    variants = [None, Variant(stage=1), Variant(stage=-1), Variant(live_map=1), Variant(live_map=-1),
                Variant(live=1), Variant(loop=-1), Variant(waves=4), Variant(waves=8),
                Variant(waves=4, live_map=1), Variant(loop=-1, live_map=-1, live=1)]
    for i in range(300):
        b = rng.choice([1, 1, 2, 3]); hk = rng.choice([1, 2, 4]); h = hk * rng.choice([1, 2, 4, 8])
        sq = rng.choice([1, 7, 33, 64, 100, 128, 255, 257, 600, 1000, 2048])
        sk = rng.choice([1, 9, 63, 64, 65, 300, 500, 1023, 1024, 1500, 2051, 4099, 9000, 16387])
        if b * h * sq * sk > 6e7:
            sk = max(1, int(6e7 // (b * h * sq)))
        d = rng.choice([64, 128]); dt = rng.choice([torch.bfloat16, torch.float16])
        er = rng.choice([0, 0, 3]); ec = rng.choice([0, 0, 0, 5, 8])
        kind = rng.choice(["rand", "causal", "bias", "window", "rows", "pad", "holes", "dense"])
        splits = rng.choice([0, 0, 0, 2, 3, 7])
        var = rng.choice(variants)
        g = torch.Generator(device=gpu).manual_seed(5000 + i)
        q = (torch.randn(b, h, sq, d, generator=g, device=gpu) * 0.6).to(dt)
        k = (torch.randn(b, hk, sk, d, generator=g, device=gpu) * 0.6).to(dt)
        v = (torch.randn(b, hk, sk, d, generator=g, device=gpu) * 0.6).to(dt)
        m = torch.zeros(b, 1, sq + er, sk + ec, device=gpu)
        r = torch.arange(sq + er, device=gpu).view(-1, 1)
        c = torch.arange(sk + ec, device=gpu).view(1, -1)
        if kind == "rand":
            m.masked_fill_(torch.rand(m.shape, generator=g, device=gpu) < 0.2, float("-inf"))
        elif kind == "causal":
            m.masked_fill_(c > r + (sk - sq), float("-inf"))
        elif kind == "bias":
            m += torch.randn(m.shape, generator=g, device=gpu) * 2.0
        elif kind == "window":
            off = r + (sk - sq)
            m.masked_fill_((c > off) | (c <= off - rng.choice([64, 300, 1000])), float("-inf"))
        elif kind == "pad":
            for bb in range(b):
                m[bb, :, :, rng.randint(0, sk):] = float("-inf")
        elif kind == "holes":
            m.masked_fill_(((c // 64) % 3 == 1) | ((c // 200) % 2 == 0), float("-inf"))
        elif kind == "rows":
            m[:, :, ::7, :] = float("-inf")
        if ec:
            m[..., sk:] = 1.0
        m = m.to(dt)
        case = dict(i=i, b=b, h=h, hk=hk, sq=sq, sk=sk, d=d, dtype=str(dt), kind=kind, er=er, ec=ec,
                    splits=splits, variant=repr(var))
        out = mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=var)
        assert_close(out, ref_attn_torch(q, k, v, m), str(case))
        dead = torch.isinf(m[:, :, :sq, :sk].float()).all(-1).squeeze(1)   # [b, sq]
        if dead.any():
            assert torch.all(out.permute(0, 2, 1, 3)[dead] == 0), str(case)


@pytest.mark.parametrize("shape", [(1, 16, 128, 32768, 128), (4, 16, 2048, 2048, 128),
                                   (2, 16, 1000, 4099, 128), (1, 4, 64, 777, 64)])
def test_num_splits_for_matches_library_plan(gpu, shape):
    """fa.num_splits_for reports the split count the launcher plans (it is the
    same C entry point, fed from the tensors)."""
    from custom_ops_amd import _lib, fa
    b, h, sq, sk, d = shape
    q = torch.zeros(b, h, sq, d, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(b, h, sk, d, dtype=torch.bfloat16, device=gpu)
    m = torch.zeros(b, 1, sq, sk, dtype=torch.bfloat16, device=gpu)
    got = fa.num_splits_for(q, k, k, m)
    p = fa.make_params(q, k, k, m, torch.empty_like(q))
    assert got == _lib.num_splits(p) >= 1
    if shape[3] == 32768:
        assert got > 1          # the small-grid long-Sk shape is split
    if shape[0] == 4:
        assert got == 1         # a grid that fills the chip is not
