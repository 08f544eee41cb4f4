"""Live-range narrowing (each workgroup runs only the KV tiles from the first to
the last one in which its rows' mask has a visible entry, and the splits share
that range): parity on masks with dead edges, for every tile-loop form, with
narrowing forced on (``Variant(live=1)``) and off (``live=-1``), and, for
masks whose rows are not 16-byte aligned, the live ranges from the pre-pass
live-tile map against each workgroup's own scan (``live_map=-1``), and the
mask read from the pre-pass's aligned staged copy (``stage=1``) against the
mask read in place (``stage=-1``).

  * every output against the fp32 torch restatement of the reference op
    (tests/test_mha_fwd_with_mask.py:38-53 of the reference) at the suite's
    tolerance, fully masked rows exactly 0;
  * unsplit launches: narrowed == not narrowed, bit for bit (a tile whose
    scores are all -inf leaves O, l and the running max unchanged);
  * split launches re-partition the live range, so only the tolerance holds;
  * the live-tile map (exact ranges) and the scan (ranges that may be wider):
    bit for bit when unsplit, within the tolerance when split.

Cases: causal, sliding window, leading + trailing key padding, an m-block
whose rows are all masked, only the last (ragged) tile live, only key 0 live,
mask rows past Sq that are visible (ignored), visible trap columns past Sk
(ignored), unaligned mask rows (Sk % 8 != 0), GQA packing, fp16, d = 64, and
forced split counts.
"""
import pytest
import torch

from tests._ref import assert_close, ref_attn_torch

NEG = float("-inf")


def mask_of(kind, b, sq, sk, skm, msq, g):
    i = torch.arange(msq).view(msq, 1)
    j = torch.arange(skm).view(1, skm)
    m = torch.zeros(b, 1, msq, skm)
    if kind == "causal":
        m.masked_fill_((j > i).expand(b, 1, msq, skm), NEG)
    elif kind == "window":
        off = sk - sq
        vis = (j <= i + off) & (j > i + off - 300)
        m.masked_fill_((~vis).expand(b, 1, msq, skm), NEG)
    elif kind == "pad":
        m[..., :500] = NEG
        m[..., sk - 1000:] = NEG
    elif kind == "dead_block":
        m[:, :, :300, :] = NEG
    elif kind == "last_tile":
        m[..., : sk - 5] = NEG
    elif kind == "first_key":
        m[..., 1:] = NEG
    elif kind == "rows_past_sq":
        m[:, :, :sq, :] = NEG
        m[:, :, :sq, sk // 2: sk // 2 + 70] = 0.0
    elif kind == "trap_cols":
        m[..., : sk - 100] = NEG
    else:
        raise ValueError(kind)
    m.masked_fill_(torch.rand(b, 1, msq, skm, generator=g) < 0.05, NEG)
    if kind == "trap_cols":
        m[..., sk:] = 0.0          # visible, but past Sk: ignored
    if kind == "rows_past_sq":
        m[:, :, sq:, :] = 0.0      # visible, but rows past Sq: ignored
    return m


CASES = [  # kind, b, h, hk, sq, sk, d, dtype, splits (0: the plan's), extra mask cols, extra mask rows
    ("causal", 1, 4, 4, 1000, 1000, 128, torch.bfloat16, 0, 0, 0),
    ("causal", 1, 4, 4, 600, 1000, 128, torch.bfloat16, 1, 0, 0),
    ("window", 2, 8, 2, 700, 2500, 128, torch.bfloat16, 1, 0, 0),
    ("window", 2, 8, 2, 700, 2500, 128, torch.bfloat16, 3, 0, 0),
    ("window", 1, 16, 4, 1000, 4099, 128, torch.bfloat16, 0, 0, 0),
    ("pad", 1, 4, 1, 300, 3000, 128, torch.bfloat16, 1, 0, 0),
    ("pad", 1, 4, 1, 300, 3000, 128, torch.bfloat16, 7, 0, 0),
    ("dead_block", 1, 2, 2, 600, 900, 128, torch.bfloat16, 1, 0, 0),
    ("dead_block", 1, 2, 2, 600, 900, 128, torch.bfloat16, 2, 0, 0),
    ("last_tile", 1, 2, 1, 256, 1029, 128, torch.bfloat16, 1, 0, 0),
    ("last_tile", 1, 2, 1, 256, 1029, 128, torch.bfloat16, 4, 0, 0),
    ("first_key", 1, 2, 2, 256, 2048, 128, torch.bfloat16, 1, 0, 0),
    ("rows_past_sq", 1, 2, 2, 200, 1024, 128, torch.bfloat16, 1, 0, 56),
    ("trap_cols", 1, 2, 2, 256, 1030, 128, torch.bfloat16, 1, 10, 0),
    ("window", 1, 4, 4, 512, 2048, 128, torch.float16, 1, 0, 0),
    ("window", 1, 4, 4, 512, 2048, 64, torch.bfloat16, 1, 0, 0),
    ("causal", 1, 4, 2, 512, 512, 64, torch.float16, 2, 0, 0),
    # rows not 16-byte aligned (the live-tile map): trap columns, rows past
    # Sq, fp16, d = 64, and batch 1's mask starting off a 16-byte boundary
    ("trap_cols", 1, 2, 2, 256, 1030, 128, torch.bfloat16, 1, 3, 0),
    ("rows_past_sq", 1, 2, 2, 200, 1021, 128, torch.bfloat16, 2, 0, 56),
    ("window", 1, 4, 4, 512, 2051, 128, torch.float16, 1, 0, 0),
    ("window", 1, 4, 4, 512, 2051, 64, torch.bfloat16, 3, 0, 0),
    ("pad", 1, 4, 1, 300, 3001, 128, torch.bfloat16, 5, 0, 0),
    ("window", 2, 4, 2, 301, 777, 128, torch.bfloat16, 0, 0, 0),
    ("causal", 2, 4, 2, 301, 777, 128, torch.bfloat16, 3, 0, 0),
]


@pytest.mark.gpu
@pytest.mark.parametrize("loop", [-1, 1, 2, 3])
def test_live_range_parity(gpu, loop):
    from custom_ops_amd import Variant, mha_fwd_with_mask
    on, off = Variant(loop=loop, live=1), Variant(loop=loop, live=-1)
    scan = Variant(loop=loop, live=1, live_map=-1)   # unaligned rows: the scan instead of the map
    # unaligned rows: the staged copy (the default) / the mask read in place
    staged, inplace = Variant(loop=loop, live=1, stage=1), Variant(loop=loop, live=1, stage=-1)
    for n, (kind, b, h, hk, sq, sk, d, dt, splits, xc, xr) in enumerate(CASES):
        g = torch.Generator().manual_seed(1000 + n)
        q = (torch.randn(b, h, sq, d, generator=g) * 0.5).to(dt).cuda()
        k = (torch.randn(b, hk, sk, d, generator=g) * 0.5).to(dt).cuda()
        v = (torch.randn(b, hk, sk, d, generator=g) * 0.5).to(dt).cuda()
        m = mask_of(kind, b, sq, sk, sk + xc, sq + xr, g).to(dt).cuda()
        ref = ref_attn_torch(q, k, v, m[:, :, :sq, :sk])
        dead = torch.isinf(m[:, :, :sq, :sk].float()).all(-1)          # [b, 1, sq]
        outs = [mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=var)
                for var in (on, off, scan, staged, inplace)]
        torch.cuda.synchronize()
        # Unsplit, the map's exact range and the scan's (which may be wider: a
        # chunk read partly past the end of the mask counts as visible) give
        # the same bits, since dead tiles add nothing; split launches then
        # partition different ranges, so only the tolerance holds.
        if splits == 1:
            assert torch.equal(outs[0].view(torch.int16), outs[2].view(torch.int16)), \
                f"loop {loop} case {n} {kind}: live-tile map and scan differ"
        for var, out in zip(("on", "off", "scan", "staged", "in place"), outs):
            tag = f"loop {loop} live {var} case {n} {kind}"
            assert_close(out, ref, tag)
            assert bool((out.float().masked_select(dead.unsqueeze(-1).expand(b, h, sq, d)) == 0).all()), tag
        if splits == 1:
            assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), \
                f"loop {loop} case {n} {kind}: narrowed unsplit launch differs"


MAP_CASES = [  # kind, b, h, hk, sq, sk, d, dtype, splits, extra mask cols, extra mask rows, waves
    ("causal", 2, 16, 4, 1000, 4099, 128, torch.bfloat16, 2, 0, 0, 8),    # last tile dead in every row block
    ("causal", 1, 4, 1, 1000, 3001, 128, torch.bfloat16, 1, 0, 0, 4),
    ("window", 2, 16, 4, 1000, 4099, 128, torch.bfloat16, 2, 0, 0, 8),
    ("window", 2, 4, 2, 301, 777, 128, torch.bfloat16, 1, 0, 0, 8),
    ("pad", 1, 4, 1, 300, 3001, 128, torch.bfloat16, 5, 0, 0, 4),
    ("trap_cols", 1, 2, 2, 256, 1030, 128, torch.bfloat16, 1, 3, 0, 8),
    ("rows_past_sq", 1, 2, 2, 200, 1021, 128, torch.float16, 2, 0, 56, 4),
    ("last_tile", 2, 4, 1, 130, 3001, 64, torch.bfloat16, 1, 0, 0, 4),
]


@pytest.mark.gpu
def test_live_map_and_staged_mask_match_host(gpu):
    """The pre-pass outputs themselves, read back from the workspace (after the
    split partials and tickets: the live-tile map, ``[B][ceil(Sq / 16)]
    [ceil(tiles / 8)]`` bytes, its whole-axis flags ``[B][ceil(Sq / 16)]``,
    then the staged mask ``[B][Sq][ceil8(Sk)]``, each rounded up to 256
    bytes), against the host: map bit t of slice r / 16 set exactly when tile
    t holds a visible entry of a row r < Sq of the slice in a column < Sk
    (slices flagged whole-axis excepted: the flag is set exactly when tile 0
    and the last tile both hold one); the staged mask equal to the mask's
    rows < Sq and columns < Sk, -inf in the padding columns. Covers the chunk that holds Sk
    in the last row of the mask, whose 16-byte load would reach past the
    buffer's end."""
    import ctypes
    from custom_ops_amd import _lib, Variant
    from custom_ops_amd.fa import make_params
    lib = _lib.load()
    r256 = lambda x: (x + 255) & ~255   # noqa: E731
    for n, (kind, b, h, hk, sq, sk, d, dt, splits, xc, xr, waves) in enumerate(MAP_CASES):
        g = torch.Generator().manual_seed(2000 + n)
        q = torch.randn(b, h, sq, d, generator=g).to(dt).cuda()
        k = torch.randn(b, hk, sk, d, generator=g).to(dt).cuda()
        m = mask_of(kind, b, sq, sk, sk + xc, sq + xr, g).to(dt).cuda()
        assert (sk + xc) % 8 != 0
        for stage in (1, -1):
            out = torch.empty_like(q)
            var = Variant(waves=waves, live=1, stage=stage)
            p = make_params(q, k, k, m, out, splits, var)
            nbytes = lib.mi355_fa_workspace_bytes(ctypes.byref(p))
            ws = torch.full((nbytes,), 0xAB, dtype=torch.uint8, device="cuda")
            p.workspace, p.workspace_bytes = ws.data_ptr(), nbytes
            err = ctypes.create_string_buffer(512)
            rc = lib.mi355_fa_fwd(ctypes.byref(p), torch.cuda.current_stream().cuda_stream, err, 512)
            assert rc == 0, err.value
            torch.cuda.synchronize()
            s_ = lib.mi355_fa_num_splits(ctypes.byref(p))
            pack = 1
            while pack * 2 <= 4 and (h // hk) % (pack * 2) == 0:
                pack *= 2
            num_m, nn, slices, skp = -(-sq // (32 * waves // pack)), -(-sk // 64), -(-sq // 16), -(-sk // 8) * 8
            row_bytes = -(-nn // 8)
            off = 0
            if s_ > 1:
                off = r256(s_ * b * h * sq * d * 2) + r256(s_ * b * h * sq * 4) + r256(b * (h // pack) * num_m * 8)
            size = b * slices * row_bytes
            map_bytes = r256(size) + r256(b * slices)
            stage_bytes = r256(b * sq * skp * 2) if stage == 1 else 0
            assert nbytes == off + map_bytes + stage_bytes, (n, nbytes, off, size, stage_bytes)
            mp = ws[off: off + size].cpu().view(b, slices, row_bytes)
            full = ws[off + r256(size): off + r256(size) + b * slices].cpu().view(b, slices)
            vis = ~torch.isinf(m[:, 0, :sq, :sk].float().cpu())
            for bb in range(b):
                for sl in range(slices):
                    rr = vis[bb, sl * 16: min(sq, sl * 16 + 16)]
                    ends = bool(rr[:, :64].any()) and bool(rr[:, (nn - 1) * 64:].any())
                    # staged: the map is complete and no slice is flagged; in
                    # place: a slice whose rows hold visible entries in tile 0
                    # and in the last tile is flagged and its bytes skipped
                    assert int(full[bb, sl]) == (0 if stage == 1 else int(ends)), (n, kind, stage, bb, sl)
                    if int(full[bb, sl]):
                        continue
                    for t in range(nn):
                        want = bool(rr[:, t * 64:(t + 1) * 64].any())
                        got = bool((int(mp[bb, sl, t // 8]) >> (t % 8)) & 1)
                        assert want == got, f"case {n} {kind} stage {stage}: batch {bb} slice {sl} tile {t}: map {got}"
            if stage == 1:
                st = ws[off + map_bytes: off + map_bytes + b * sq * skp * 2].view(dt).cpu().view(b, sq, skp)
                want = torch.full((b, sq, skp), NEG, dtype=dt)
                want[:, :, :sk] = m[:, 0, :sq, :sk].cpu()
                assert torch.equal(st.view(torch.int16), want.view(torch.int16)), f"case {n} {kind}: staged mask"


@pytest.mark.gpu
def test_live_map_on_aligned_split_launches(gpu):
    """Aligned masks: the map serves 8-wave split launches by default and the
    4-wave deep ones (split-KV decode shapes) when forced
    (``Variant(live_map=1)``: the map-only kernel instance); every output
    against the fp32 restatement, and the map's ranges against the scan's
    (``live_map=-1``) within the tolerance (split launches partition them)."""
    from custom_ops_amd import Variant, mha_fwd_with_mask
    cases = [  # kind, b, h, hk, sq, sk, waves, splits
        ("causal", 1, 8, 8, 128, 8192, 4, 8),
        ("pad", 1, 8, 2, 128, 8192, 4, 16),
        ("window", 2, 8, 2, 700, 4096, 8, 2),
        ("causal", 2, 8, 8, 500, 4096, 8, 3),
    ]
    for n, (kind, b, h, hk, sq, sk, waves, splits) in enumerate(cases):
        g = torch.Generator().manual_seed(3000 + n)
        q = (torch.randn(b, h, sq, 128, generator=g) * 0.5).bfloat16().cuda()
        k = (torch.randn(b, hk, sk, 128, generator=g) * 0.5).bfloat16().cuda()
        v = (torch.randn(b, hk, sk, 128, generator=g) * 0.5).bfloat16().cuda()
        m = mask_of(kind, b, sq, sk, sk, sq, g).bfloat16().cuda()
        ref = ref_attn_torch(q, k, v, m)
        dead = torch.isinf(m.float()).all(-1)
        for label, var in (("map", Variant(waves=waves, live_map=1)), ("default", Variant(waves=waves)),
                           ("scan", Variant(waves=waves, live_map=-1))):
            out = mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=var)
            torch.cuda.synchronize()
            tag = f"case {n} {kind} {label}"
            assert_close(out, ref, tag)
            assert bool((out.float().masked_select(dead.unsqueeze(-1).expand(b, h, sq, 128)) == 0).all()), tag


@pytest.mark.gpu
def test_local_scan_keeps_split_results(gpu):
    """The compiled kernel's split launches without a map narrow each split's
    own share and keep the nominal partition: every split runs the same live
    tiles as without narrowing, so the outputs are bit for bit those of
    ``live=-1``."""
    from custom_ops_amd import Variant, mha_fwd_with_mask
    on, off = Variant(loop=-1, live=1, live_map=-1), Variant(loop=-1, live=-1)
    for n, (kind, b, h, hk, sq, sk, d, dt, splits, xc, xr) in enumerate(CASES):
        if splits <= 1:
            continue
        g = torch.Generator().manual_seed(4000 + n)
        q = (torch.randn(b, h, sq, d, generator=g) * 0.5).to(dt).cuda()
        k = (torch.randn(b, hk, sk, d, generator=g) * 0.5).to(dt).cuda()
        v = (torch.randn(b, hk, sk, d, generator=g) * 0.5).to(dt).cuda()
        m = mask_of(kind, b, sq, sk, sk + xc, sq + xr, g).to(dt).cuda()
        a = mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=on)
        c = mha_fwd_with_mask(q, k, v, m, num_splits=splits, variant=off)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), c.view(torch.int16)), f"case {n} {kind}"
        assert_close(a, ref_attn_torch(q, k, v, m[:, :, :sq, :sk]), f"case {n} {kind}")
