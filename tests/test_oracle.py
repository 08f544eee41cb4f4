"""CPU tests that pin the oracle (oracle/fa_oracle.c + oracle/oracle.py).

Each restated function is checked against something it does not share code
with: the committed golden fixtures (float64 closed form made by
tests/golden/make_golden.py), textbook special cases, invariants, and
hand-derived values of the reference's cost model.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.golden import load_fixtures

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


def rand_case(seed, B=1, H=2, Hk=2, Sq=20, Sk=37, d=64, p_inf=0.2, dtype="bf16"):
    rng = np.random.default_rng(seed)
    q = orc.round_to(rng.standard_normal((B, H, Sq, d)).astype(np.float32) * 0.5, dtype)
    k = orc.round_to(rng.standard_normal((B, Hk, Sk, d)).astype(np.float32) * 0.5, dtype)
    v = orc.round_to(rng.standard_normal((B, Hk, Sk, d)).astype(np.float32) * 0.5, dtype)
    m = np.where(rng.random((B, 1, Sq, Sk)) < p_inf, -np.inf, 0.0).astype(np.float32)
    return q, k, v, m


# ── golden fixtures ───────────────────────────────────────────────────────────
@pytest.mark.parametrize("fx", load_fixtures(), ids=lambda f: f.name)
def test_oracle_vs_golden(fx):
    q, k, v, m = fx.tensors_f32()
    exp = fx.expected
    for splits in (1, 3):
        out = orc.oracle_fwd(q, k, v, m, dtype=fx.dtype, num_splits=splits, block_n=16)
        err = np.abs(out - exp)
        assert np.all(err <= 2e-2 + 2e-2 * np.abs(exp)), f"{fx.name} s={splits}: {err.max()}"
    # without P rounding the oracle is an fp32 evaluation of the same closed form
    out32 = orc.oracle_fwd(q, k, v, m, dtype="fp32")
    assert np.abs(out32 - exp).max() < 2e-5
    for r in fx.masked_rows:
        assert np.all(out32[:, :, r] == 0)
    assert np.abs(orc.attn_fp64(q, k, v, m) - exp).max() < 1e-6
    assert np.abs(orc.ref_attn_np(q, k, v, m, "fp32") - exp).max() < 2e-5


def test_fixture_contents_sane():
    fxs = load_fixtures()
    assert len(fxs) >= 10
    names = {f.name for f in fxs}
    for must in ("allmasked_fp16_d64", "trap_bf16_d64", "sk7_fp16_d128", "gqa4_bf16_d64",
                 "sq1_fp16_d64"):
        assert must in names
    for f in fxs:
        assert np.isfinite(f.expected).all()


# ── closed-form special cases ─────────────────────────────────────────────────
def test_zero_mask_equals_plain_softmax_attention():
    q, k, v, _ = rand_case(1)
    m = np.zeros((1, 1, 20, 37), np.float32)
    s = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), k.astype(np.float64)) / 8.0
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("bhqk,bhkd->bhqd", p, v.astype(np.float64))
    assert np.abs(orc.oracle_fwd(q, k, v, m, dtype="fp32") - ref).max() < 1e-5


def test_single_visible_column_selects_v_row():
    q, k, v, _ = rand_case(2)
    m = np.full((1, 1, 20, 37), -np.inf, np.float32)
    cols = [(5 * i + 3) % 37 for i in range(20)]
    for i, c in enumerate(cols):
        m[0, 0, i, c] = 0.0
    for dtype in ("fp32", "bf16"):
        out = orc.oracle_fwd(q, k, v, m, dtype=dtype, num_splits=2, block_n=8)
        for i, c in enumerate(cols):
            assert np.array_equal(out[0, :, i], v[0, :, c])


def test_fully_masked_rows_are_zero_all_paths():
    q, k, v, m = rand_case(3)
    m[0, 0, 4] = -np.inf
    for s in (1, 2, 5):
        out = orc.oracle_fwd(q, k, v, m, dtype="bf16", num_splits=s, block_n=8)
        assert np.all(out[0, :, 4] == 0) and np.isfinite(out).all()
    assert np.all(orc.attn_fp64(q, k, v, m)[0, :, 4] == 0)
    assert np.all(orc.ref_attn_np(q, k, v, m)[0, :, 4] == 0)


def test_row_shift_invariance():
    q, k, v, m = rand_case(4, p_inf=0.1)
    shift = np.arange(20, dtype=np.float32).reshape(1, 1, 20, 1) * 0.75
    a = orc.oracle_fwd(q, k, v, m, dtype="fp32")
    b = orc.oracle_fwd(q, k, v, m + shift, dtype="fp32")
    assert np.abs(a - b).max() < 1e-5


def test_finite_bias_is_added_after_scaling():
    """softmax(S·scale + bias), not softmax((S + bias)·scale): the reference
    authors' scale-bug detector (docs/fa_sm120_porting_and_optimization.md:337)."""
    rng = np.random.default_rng(5)
    q, k, v, _ = rand_case(5, d=128)
    bias = (rng.standard_normal((1, 1, 20, 37)) * 2).astype(np.float32)
    out = orc.oracle_fwd(q, k, v, bias, dtype="fp32")
    right = orc.attn_fp64(q, k, v, bias)
    wrong = orc.attn_fp64(q, k, v, bias / np.sqrt(128))   # (S + bias)·scale
    assert np.abs(out - right).max() < 1e-5
    assert np.abs(out - wrong).max() > 1e-2


def test_gqa_equals_repeat_interleave():
    q, k, v, m = rand_case(6, H=4, Hk=1)
    a = orc.oracle_fwd(q, k, v, m, dtype="bf16")
    b = orc.oracle_fwd(q, np.repeat(k, 4, 1), np.repeat(v, 4, 1), m, dtype="bf16")
    assert np.array_equal(a, b)
    # and the GQA head mapping is h // (H/Hk), not h % Hk
    q2, k2, v2, m2 = rand_case(7, H=4, Hk=2)
    out = orc.oracle_fwd(q2, k2, v2, m2, dtype="fp32")
    ref = orc.attn_fp64(q2, np.repeat(k2, 2, 1), np.repeat(v2, 2, 1), m2)
    assert np.abs(out - ref).max() < 1e-5


def test_split_invariance_and_combine():
    q, k, v, m = rand_case(8, Sk=200, p_inf=0.3)
    m[0, 0, 2] = -np.inf
    m[0, 0, 3, :150] = -np.inf        # row visible only in the last split(s)
    base = orc.oracle_fwd(q, k, v, m, dtype="fp32", block_n=16)
    for s in (2, 3, 7, 13, 64):
        out = orc.oracle_fwd(q, k, v, m, dtype="fp32", block_n=16, num_splits=s)
        assert np.abs(out - base).max() < 1e-5, s
        assert np.all(out[0, :, 2] == 0)


def test_autopad_equivalence():
    """Sk % 8 != 0 equals the explicitly padded call (K/V zero rows, mask -inf
    columns) — the reference's auto-pad contract (csrc/fa/fa_fwd_op.cu:117-134)."""
    q, k, v, m = rand_case(9, Sk=37)
    kp = np.concatenate([k, np.zeros((1, 2, 3, 64), np.float32)], 2)
    vp = np.concatenate([v, np.zeros((1, 2, 3, 64), np.float32)], 2)
    mp = np.concatenate([m, np.full((1, 1, 20, 3), -np.inf, np.float32)], 3)
    a = orc.oracle_fwd(q, k, v, m, dtype="bf16", block_n=16)
    b = orc.oracle_fwd(q, kp, vp, mp, dtype="bf16", block_n=16)
    assert np.array_equal(a, b)


def test_trap_columns_ignored():
    q, k, v, m = rand_case(10, Sk=37)
    trap = np.concatenate([m, np.full((1, 1, 20, 11), 5.0, np.float32)], 3)
    trap = np.concatenate([trap, np.full((1, 1, 4, 48), 3.0, np.float32)], 2)
    a = orc.oracle_fwd(q, k, v, m, dtype="fp32")
    b = orc.oracle_fwd(q, k, v, trap, dtype="fp32")
    assert np.array_equal(a, b)


def test_brute_force_tiny():
    """Pure-Python loops on a 3x5 problem, no numpy linear algebra."""
    import math
    q, k, v, m = rand_case(11, H=1, Hk=1, Sq=3, Sk=5, d=64, p_inf=0.3)
    m[0, 0, 0, :] = -np.inf
    out = orc.oracle_fwd(q, k, v, m, dtype="fp32")
    for i in range(3):
        s = []
        for j in range(5):
            dot = sum(float(q[0, 0, i, t]) * float(k[0, 0, j, t]) for t in range(64))
            s.append(dot / 8.0 + float(m[0, 0, i, j]))
        mx = max(s)
        if mx == -math.inf:
            assert np.all(out[0, 0, i] == 0)
            continue
        e = [math.exp(x - mx) for x in s]
        tot = sum(e)
        for t in range(64):
            ref = sum(e[j] / tot * float(v[0, 0, j, t]) for j in range(5))
            assert abs(out[0, 0, i, t] - ref) < 1e-5


def test_p_rounding_matters_and_is_bounded():
    q, k, v, m = rand_case(12, Sk=300)
    a = orc.oracle_fwd(q, k, v, m, dtype="bf16")
    b = orc.oracle_fwd(q, k, v, m, dtype="fp32")
    d = np.abs(a - b).max()
    assert 0 < d < 2e-2


# ── rounding helpers ──────────────────────────────────────────────────────────
def test_rounding_matches_torch():
    import torch
    rng = np.random.default_rng(13)
    x = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1e-30, 65504.0, 65519.0, 3.0e-8], np.float32)])
    bf = torch.from_numpy(x).bfloat16().float().numpy()
    hf = torch.from_numpy(x).half().float().numpy()
    assert np.array_equal(orc.round_to(x, "bf16"), bf)
    for i in range(0, len(x), 97):
        assert orc.oracle_round_scalar(float(x[i]), "bf16") == bf[i]
        assert orc.oracle_round_scalar(float(x[i]), "fp16") == hf[i]


# ── reference cost model (csrc/fa/fa_fwd_launch.h:137-170) ─────────────────────
def test_cost_model_reference_values():
    """Hand-derived for the sm89 constants (K = 2.25, P0 = 0.35, d128 M64 tiles):
    config 4 (B1 H16 Sq128 Sk32768 → 32 m-blocks, 512 n-blocks) gives 8 splits on
    a 128-SM RTX 4090D and 16 on 256 CUs; large grids never split."""
    assert orc.oracle_num_splits(32, 512, 64, 128, 128, 2.25) == 8
    assert orc.oracle_num_splits(32, 512, 64, 128, 256, 2.25) == 16
    assert orc.oracle_num_splits(2048, 32, 64, 128, 128, 2.25) == 1   # cfg2-sized grid
    assert orc.oracle_num_splits(4, 4, 64, 128, 128, 2.25) == 1       # nb <= 4
    # B1 H1 Sq128 Sk32768 on 4090D: 2 m-blocks, cap_fill 128 → s* = sqrt(512·2.25/0.35)
    s_star = int(np.sqrt(512 * 2.25 / 0.35))
    s = orc.oracle_num_splits(2, 512, 64, 128, 128, 2.25)
    assert s_star - 8 <= s <= min(64, s_star + 8)
    costs = {c: -(-512 // c) * 2.25 + c * 0.35 for c in range(max(1, s_star - 8),
                                                              min(64, s_star + 8) + 1)}
    assert s == min(costs, key=lambda c: (costs[c], c))


def test_torch_math_cpu_matches_closed_form():
    import torch
    q, k, v, m = rand_case(14, H=4, Hk=2)
    t = [torch.from_numpy(a) for a in (q, k, v, m)]
    out = orc.torch_math_cpu(*t).numpy()
    assert np.abs(out - orc.attn_fp64(q, k, v, m)).max() < 1e-5
