"""CPU tests of the host side: the C-ABI library loads and exports every symbol
include/mi355_fa.h declares, its validation and cost model behave, and the
torch op / facade mirror the reference's contract (no GPU calls)."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mi355_fa.h")


@pytest.fixture(scope="module")
def lib():
    from custom_ops_amd import _lib
    return _lib.load()


def header_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mi355_fa_\w+)\s*\(", src)))


def test_header_symbols_exported(lib):
    from custom_ops_amd import _lib
    names = header_functions()
    assert set(names) == set(_lib.EXPORTED)
    for n in names:
        assert hasattr(lib, n), f"{n} not exported"
    assert lib.mi355_fa_abi_version() == _lib.ABI_VERSION == 3
    assert b"gfx950" in lib.mi355_fa_build_info()


def _struct_fields(src, name):
    body = src[src.index(f"typedef struct {name}"):src.index(f"}} {name};")]
    fields = []
    for line in body.splitlines()[1:]:
        line = line.strip().rstrip(";")
        if not line:
            continue
        # "<type> a, b, c" or "<type>* a": the names are the last word of each part
        fields += [re.findall(r"\w+", part)[-1] for part in line.split(",")]
    return fields


def test_params_struct_layout_matches_header():
    """ctypes mirrors have the header's field order; sizes are multiples of 8 / 4."""
    from custom_ops_amd import _lib
    src = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    assert [f[0] for f in _lib.Params._fields_] == _struct_fields(src, "mi355_fa_params")
    assert [f[0] for f in _lib.Variant._fields_] == _struct_fields(src, "mi355_fa_variant")
    assert ctypes.sizeof(_lib.Params) % 8 == 0
    assert ctypes.sizeof(_lib.Variant) == 4 * len(_lib.Variant._fields_)
    assert _lib.Params.variant.offset == ctypes.sizeof(_lib.Params) - 8


def _params(**kw):
    from custom_ops_amd import _lib
    p = _lib.Params()
    p.q = p.k = p.v = p.mask = p.o = 0x10000
    p.b, p.h, p.h_k, p.seqlen_q, p.seqlen_k, p.d = 1, 4, 2, 128, 256, 128
    p.mask_seqlen_q, p.mask_seqlen_k = 128, 256
    p.q_row_stride = p.k_row_stride = p.v_row_stride = p.o_row_stride = 128
    p.mask_row_stride = 256
    p.dtype = _lib.BF16
    p.scale_softmax = 128 ** -0.5
    for key, val in kw.items():
        setattr(p, key, val)
    return p


@pytest.mark.parametrize("field,value,msg", [
    ("d", 96, "head_dim=64 or head_dim=128"),
    ("dtype", 7, "float16 or bfloat16"),
    ("h_k", 3, "divisible by n_kv_heads"),
    ("h_k", 0, "divisible by n_kv_heads"),
    ("mask_seqlen_q", 100, "mask shape"),
    ("o_row_stride", 132, "multiples of 8 elements"),   # O leaves in 16-byte row chunks
    ("mask_seqlen_k", 255, "mask shape"),
    ("scale_softmax", -1.0, "scale_softmax"),
    ("q", 0, "NULL"),
    ("q_row_stride", 129, "aligned"),
])
def test_c_abi_validation(lib, field, value, msg):
    from custom_ops_amd import _lib
    p = _params(**{field: value})
    err = ctypes.create_string_buffer(256)
    rc = lib.mi355_fa_fwd(ctypes.byref(p), None, err, 256)
    assert rc == _lib.EINVAL
    assert msg in err.value.decode()


def test_c_abi_empty_problem_is_noop(lib):
    p = _params(b=0)
    err = ctypes.create_string_buffer(64)
    assert lib.mi355_fa_fwd(ctypes.byref(p), None, err, 64) == 0


def test_cost_model_and_workspace(lib):
    from custom_ops_amd import _lib
    # reference-shaped inputs reproduce the reference's hand-derived split counts
    assert _lib.cost_model_splits(32, 512, 64, 128, 128) == 8
    assert _lib.cost_model_splits(32, 512, 64, 128, 256) == 16
    assert _lib.cost_model_splits(1024, 32, 128, 128, 256) == 1
    # the library's own tiling (BM=128): identical to the reference formula
    from oracle import oracle as orc
    for tot, nb, cus in [(16, 512, 256), (2, 128, 256), (64, 1024, 256), (8, 5, 256),
                         (200, 64, 256), (1, 513, 80)]:
        assert _lib.cost_model_splits(tot, nb, 128, 128, cus) == \
            orc.oracle_num_splits(tot, nb, 128, 128, cus, 2.25)
        assert _lib.cost_model_splits(tot, nb, 128, 64, cus) == \
            orc.oracle_num_splits(tot, nb, 128, 64, cus, 2.5)
    # forced splits are clamped to [1, min(64, n_blocks)]; workspace covers partials
    p = _params(num_splits=200, seqlen_k=64 * 100, mask_seqlen_k=64 * 100)
    assert _lib.num_splits(p) == 64
    rows = 64 * 1 * 4 * 128
    assert _lib.workspace_bytes(p) >= rows * 128 * 2 + rows * 4   # 16-bit O partials + fp32 LSE
    p = _params(num_splits=1)
    assert _lib.num_splits(p) == 1 and _lib.workspace_bytes(p) == 0



def test_workspace_of_masks_with_unaligned_rows(lib):
    """The workspace of a mask whose rows are not 16-byte aligned: the
    live-tile map ([B][ceil(Sq/16)][ceil(tiles/8)] bytes) and its whole-axis
    flags ([B][ceil(Sq/16)]), then the staged copy ([B][Sq][ceil8(Sk)] 16-bit
    entries), each rounded up to 256 bytes; Variant(stage=-1) drops the copy,
    Variant(live_map=-1) the map; an aligned unsplit launch needs none."""
    from custom_ops_amd import _lib
    r256 = lambda x: (x + 255) & ~255   # noqa: E731
    for b, sq, sk in [(1, 128, 259), (2, 1000, 4099), (3, 17, 777)]:
        common = dict(b=b, seqlen_q=sq, mask_seqlen_q=sq, seqlen_k=sk, mask_seqlen_k=sk,
                      mask_row_stride=sk, num_splits=1)
        slices, groups, skp = -(-sq // 16), -(-(-(-sk // 64)) // 8), -(-sk // 8) * 8
        map_bytes = r256(b * slices * groups) + r256(b * slices)
        staged = r256(b * sq * skp * 2)
        assert _lib.workspace_bytes(_params(**common)) == map_bytes + staged, (b, sq, sk)
        v = _lib.Variant(stage=-1)
        assert _lib.workspace_bytes(_params(variant=ctypes.pointer(v), **common)) == map_bytes
        v2 = _lib.Variant(live_map=-1)
        assert _lib.workspace_bytes(_params(variant=ctypes.pointer(v2), **common)) == staged
    aligned = dict(seqlen_k=264, mask_seqlen_k=264, mask_row_stride=264, num_splits=1)
    assert _lib.workspace_bytes(_params(**aligned)) == 0


@pytest.mark.parametrize("b,h,sq,sk,d,splits", [
    # configurations of the benchmark (all agree with the measured best)
    (4, 16, 2048, 2048, 128, 1),      # cfg2: 512 workgroups of 8 waves, two rounds
    (1, 16, 128, 32768, 128, 16),     # cfg4: 256 workgroups of 4 waves, one each
    (2, 16, 1000, 4099, 128, 2),      # cfg5
    (1, 16, 512, 32768, 128, 8),
    (1, 64, 1, 32768, 64, 8),
    (1, 4, 512, 32768, 128, 32),
    (1, 4, 512, 8192, 128, 16),
    (1, 1, 1, 256, 128, 1),           # >= 4 KV tiles per split caps the count
    (1, 1, 1, 1024, 128, 4),
    # the measured best in the sweeps the model was fitted to, where filling
    # one round of CUs chose otherwise (hot µs: model's plan vs that rule's)
    (1, 64, 1, 8192, 128, 8),         # 39.4 vs 48.9 (4 splits)
    (1, 16, 1, 32768, 128, 32),       # 42.4 vs 49.7 (16 splits)
    (1, 16, 128, 8192, 64, 16),       # 18.5 vs 20.6 (32 splits)
    (1, 32, 1024, 1024, 64, 1),       # 18.9 vs 23.9 (2 splits)
    (1, 16, 1536, 4099, 128, 5),      # 85.2 vs 114.8 (8 waves, 3 splits: 288 workgroups,
                                      # a second round of 32)
])
def test_auto_plan_fills_whole_rounds(lib, b, h, sq, sk, d, splits):
    """The launcher's own plan on a 256-CU part (no GPU here: the library
    assumes 256 CUs when none can be queried), from its occupancy cost model."""
    from custom_ops_amd import _lib
    p = _params(b=b, h=h, h_k=h, seqlen_q=sq, seqlen_k=sk, d=d, mask_seqlen_q=sq,
                mask_seqlen_k=sk, q_row_stride=d, k_row_stride=d, v_row_stride=d,
                o_row_stride=d, mask_row_stride=sk)
    assert _lib.num_splits(p) == splits


def test_torch_op_schema_and_fake():
    import custom_ops_amd
    custom_ops_amd.ops.ensure_loaded()
    op = torch.ops.recsys_ops.mha_fwd_with_mask
    sch = str(op.default._schema)
    assert sch == "recsys_ops::mha_fwd_with_mask(Tensor q, Tensor k, Tensor v, Tensor mask) -> Tensor"
    q = torch.empty(2, 8, 100, 128, dtype=torch.bfloat16, device="meta")
    k = torch.empty(2, 2, 77, 128, dtype=torch.bfloat16, device="meta")
    m = torch.empty(2, 1, 100, 77, dtype=torch.bfloat16, device="meta")
    out = op(q, k, k, m)
    assert out.shape == q.shape and out.dtype == q.dtype and out.device.type == "meta"


def test_cpu_tensors_rejected_like_reference():
    from custom_ops_amd import ops
    x = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16)
    m = torch.zeros(1, 1, 8, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="only supported on CUDA"):
        ops.mha_fwd_with_mask(x, x, x, m)


def test_backend_selection():
    from custom_ops_amd import _resolve_backend, ops
    assert _resolve_backend(None) in ("auto", "cuda", "hip")
    with pytest.raises(RuntimeError, match="Tile-lang"):
        _resolve_backend("tilelang")
    with pytest.raises(ValueError):
        _resolve_backend("bogus")
    with pytest.raises(AttributeError, match="No op 'nope'"):
        ops.nope
    assert ops.groups["fa"] in ("loaded", "not_loaded", "failed")


def test_validation_messages_on_host():
    """The Python layer's checks (run before any device work) follow the
    reference's order and text (csrc/fa/fa_fwd_op.cu:53-108)."""
    from custom_ops_amd import fa

    class Fake:
        def __init__(self, shape, dtype=torch.bfloat16, contig=True, dev=0, cuda=True):
            self.shape, self.dtype, self._c = torch.Size(shape), dtype, contig
            self.is_cuda, self.device = cuda, torch.device("cuda", dev)

        def get_device(self):
            return self.device.index if self.is_cuda else -1

        def is_contiguous(self):
            return self._c

        def dim(self):
            return len(self.shape)

    q = Fake((1, 4, 8, 64))
    k = Fake((1, 2, 8, 64))
    m = Fake((1, 1, 8, 8))
    fa.validate(q, k, k, m)
    cases = [
        ((Fake((1, 4, 8, 64), torch.float32), k, k, Fake((1, 1, 8, 8), torch.float32)),
         "float16 or bfloat16"),
        ((q, Fake((1, 2, 8, 64), torch.float16), k, m), "k dtype must match q"),
        ((q, k, k, Fake((1, 1, 8, 8), torch.float16)), "mask dtype must match q"),
        ((Fake((1, 4, 8, 64), contig=False), k, k, m), "q must be contiguous"),
        ((Fake((4, 8, 64)), k, k, m), "q must be 4D"),
        ((q, Fake((2, 2, 8, 64)), k, m), "Batch size mismatch"),
        ((q, Fake((1, 2, 8, 32)), k, m), "head_dim mismatch"),
        ((q, k, Fake((1, 2, 9, 64)), m), "seqlen_k mismatch"),
        ((q, Fake((1, 3, 8, 64)), Fake((1, 3, 8, 64)), m), "divisible"),
        ((Fake((1, 4, 8, 96)), Fake((1, 2, 8, 96)), Fake((1, 2, 8, 96)), m), "head_dim=64"),
        ((q, k, k, Fake((1, 2, 8, 8))), "mask shape"),
        ((q, k, k, Fake((1, 1, 7, 8))), "mask shape"),
        ((q, k, k, Fake((1, 1, 8, 7))), "mask shape"),
        ((q, k, k, Fake((1, 1, 8, 8), cuda=False)), "mask must be a CUDA tensor"),
        ((q, k, k, Fake((1, 1, 8, 8), dev=1)), "same device"),
        ((q, k, Fake((1, 2, 8, 64), contig=False), m), "v must be contiguous"),
        ((q, k, k, Fake((1, 1, 8, 8, 1))), "mask must be 4D"),
        ((q, Fake((1, 0, 8, 64)), Fake((1, 0, 8, 64)), m), "divisible"),
        ((q, k, Fake((1, 4, 8, 64)), m), "n_kv_heads mismatch between k/v"),
    ]
    assert fa._valid(q, k, k, m)
    for args, msg in cases:
        # the one-expression fast path rejects exactly what the ordered checks reject
        assert not fa._valid(*args), msg
        with pytest.raises(RuntimeError, match=msg):
            fa.validate(*args)


def test_workloads_match_baseline_configs():
    import json
    from custom_ops_amd.workloads import CONFIGS, make_mask
    base = json.load(open(os.path.join(ROOT, "BASELINE.json")))
    assert len(base["configs"]) == 5
    c2, c4, c5 = CONFIGS["cfg2"], CONFIGS["cfg4"], CONFIGS["cfg5"]
    assert (c2.B, c2.H, c2.Hk, c2.Sq, c2.Sk, c2.d) == (4, 16, 16, 2048, 2048, 128)
    assert (CONFIGS["cfg3"].Hk) == 4
    assert (c4.B, c4.H, c4.Sq, c4.Sk) == (1, 16, 128, 32768)
    assert (c5.B, c5.H, c5.Hk, c5.Sq, c5.Sk) == (2, 16, 4, 1000, 4099)
    assert abs(c2.flops - 137.44e9) < 0.01e9
    g = torch.Generator().manual_seed(0)
    m = make_mask("random10_diag", 1, 256, 256, g)
    assert torch.all(torch.diagonal(m[0, 0]) == 0)
    frac = torch.isinf(m).float().mean().item()
    assert 0.08 < frac < 0.12
    m5 = make_mask("window_pad_random5", 2, 100, 1400, g)
    assert torch.all(torch.isinf(m5[1, 0, :, 1100:]))
    vis = ~torch.isinf(m5[0, 0])
    assert vis.sum(-1).max() <= 1024
