"""Tile plans (vrs_model_get_plan / vrs_model_set_plan), the fp8-forced
autotune mode and vrs_model_conv_io, through the C ABI."""
import numpy as np
import pytest

from gpu_util import bf16_round, ctx, dev, vrs
from golden_io import seeded_params

pytestmark = pytest.mark.gpu


def _yolo(batch, size, dtype, autotune=True):
    desc = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="m", one2one=True)
    return vrs.Model(ctx(), desc, batch, size, size, dtype, 1e-3, autotune=autotune)


def _params(m):
    P = seeded_params(m.params(), 0, bn="random")
    return {k: (bf16_round(v) if v.ndim == 4 else v) for k, v in P.items()}


def test_plan_round_trip_bit_identical():
    """An autotuned model's plan applied to a fresh model gives the same plan
    and bit-identical outputs; a failed finalize (bad plan) leaves the model
    usable with a good plan."""
    import torch
    m1 = _yolo(2, 256, vrs.BF16)
    P = _params(m1)
    m1.load(P)
    plan = m1.get_plan()
    assert len(plan) == len(m1.conv_info()) and any(plan)
    x = dev(np.random.default_rng(3).uniform(0, 1, (2, 3, 256, 256)).astype(np.float32))
    o1 = [o.clone() for o in m1.forward(x)]
    m2 = _yolo(2, 256, vrs.BF16)
    # a bad plan first: a persistent tile on a conv with a residual
    # (model.2.m.0.cv2), which those kernels do not take
    names = [pre for pre, _, _ in m2.conv_info()]
    bad = list(plan)
    bad[names.index("model.2.m.0.cv2")] = vrs.TILE_128x128 | vrs.TILE_K32 | vrs.TILE_PERSIST
    m2.set_plan(bad)
    with pytest.raises(vrs.VrsError) as e:
        m2.load(P)
    assert "model.2.m.0.cv2" in str(e.value)
    m2.set_plan(plan)
    m2.load(P)   # the parameters are still there: finalize retried with a valid plan
    assert m2.get_plan() == plan
    o2 = m2.forward(x)
    torch.cuda.synchronize()
    for a, b in zip(o1, o2):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_plan_rejections():
    m = _yolo(1, 128, vrs.BF16)
    n = len(m.conv_info())
    with pytest.raises(vrs.VrsError):
        m.set_plan([0] * (n - 1))        # wrong length
    names = [pre for pre, _, _ in m.conv_info()]
    bad = [0] * n
    bad[names.index("model.23.one2one_cv3.0.0.0")] = vrs.TILE_128x128   # depthwise: takes no tile
    m.set_plan(bad)
    with pytest.raises(vrs.VrsError):
        m.load(_params(m))
    bad = [0] * n
    bad[names.index("model.3")] = vrs.TILE_128x128 | vrs.PLAN_FP8       # fp8 in a bf16 model
    m2 = _yolo(1, 128, vrs.BF16)
    m2.set_plan(bad)
    with pytest.raises(vrs.VrsError):
        m2.load(_params(m2))
    with pytest.raises(vrs.VrsError):
        _yolo(1, 128, vrs.BF16, autotune=2)   # mode 2 is for fp8 models


def test_fp8_forced_mode_keeps_every_eligible_conv_on_fp8():
    import torch
    m = _yolo(2, 256, vrs.FP8, autotune=2)
    m.load(_params(m))
    x = dev(np.random.default_rng(4).uniform(0, 1, (2, 3, 256, 256)).astype(np.float32))
    m.calibrate(x)
    m.forward(x)
    torch.cuda.synchronize()
    ios = [m.conv_io(i) for i in range(len(m.conv_info()))]
    eligible = [io for io in ios if io.groups == 1 and not io.stem and io.cin % 64 == 0 and
                (io.up.data is None or io.up.c % 64 == 0)]
    assert all(io.fp8 for io in eligible) and len(eligible) > 60
    assert any(io.up.data is not None for io in eligible)   # the fused-upsample convs too
    plan = m.get_plan()
    # every eligible conv has an fp8 plan entry, the Detect output convs included
    assert sum(1 for p in plan if p & vrs.PLAN_FP8) == len(eligible)
    assert all(io.in_scale > 0 for io in eligible)
    # e4m3 storage: inputs read as e4m3 use their buffer's step; buffers with
    # a non-fp8 reader or writer (attention, SPPF, depthwise, the stem) stay bf16
    x8 = [io for io in eligible if io.x_e4m3]
    assert len(x8) > 30 and all(io.in_scale == io.x_step for io in x8)
    assert sum(io.y_e4m3 for io in ios) > 30
    for i, (pre, _, _) in enumerate(m.conv_info()):
        if pre.endswith(("attn.qkv", "model.9.cv1", "model.16.cv2")) or ".one2one_cv3." in pre and pre.endswith(".0"):
            assert not ios[i].y_e4m3, pre


def test_conv_io_views():
    """conv_io describes each conv: launch order, views inside the model's
    buffers, the stem and the flat Detect outputs."""
    import torch
    m = _yolo(1, 128, vrs.BF16, autotune=False)
    m.load(_params(m))
    m.forward(dev(np.zeros((1, 3, 128, 128), np.float32)))
    torch.cuda.synchronize()
    info = m.conv_info()
    names = m.launch_names()
    seen = set()
    for i, (pre, _, _) in enumerate(info):
        io = m.conv_io(i)
        if pre.endswith(".pe"):            # parameters of the fused attention launch
            assert io.launch == -1
            continue
        assert 0 <= io.launch < len(names) and names[io.launch].startswith(pre + ":")
        assert io.launch not in seen
        seen.add(io.launch)
        if pre == "model.0":
            assert io.stem and io.x.data is None and io.y.data is not None
        elif pre.endswith(".2") and "one2one" in pre:
            assert io.y.data is None and io.out_idx in (0, 1) and io.plain
        else:
            assert io.x.data is not None and io.y.data is not None and io.x.c == io.cin
    with pytest.raises(vrs.VrsError):
        m.conv_io(len(info))


def test_leftover_tiles_run_on_the_128x128_tile():
    """A 256x256-tile conv whose tiles leave the last round at most half full
    (3x3/s2 256->256, 68 images of 64x64: 272 tiles on 256 CUs) runs its full
    rounds on the 256x256 tile and the 16 leftover pixel tiles on the
    128x128 k64 tile.  Both accumulate each output over K in the same step
    order, so the result is bit-identical to the whole conv on the 128x128
    tile; and within the bf16 bar of the oracle on the last two images (the
    leftover tiles)."""
    import torch
    import oracle
    from gpu_util import from_nhwc, rel_err, to_nhwc
    TOL, FLOOR = 2e-2, 1e-1   # the bf16 single-kernel bar (elementwise, floor 0.1 * rms)
    B, S = 68, 64
    desc = vrs.block(vrs.BLOCK_CONV, 256, 256, k=3, s=2)
    m = vrs.Model(ctx(), desc, B, S, S, vrs.BF16, 1e-3, autotune=False)
    m.set_plan([vrs.TILE_256x256] * len(m.conv_info()))
    P = _params(m)
    m.load(P)
    x = bf16_round(np.random.default_rng(5).standard_normal((B, 256, S, S)).astype(np.float32))
    xd = dev(x)
    out = m.forward(xd)[0]
    torch.cuda.synchronize()
    names = m.launch_names()
    i256 = [k for k, n in enumerate(names) if n.endswith("vrs_conv_bf16_256x256_k64_a")]
    assert len(i256) == 1 and names[i256[0] + 1].endswith("vrs_conv_bf16_128x128_k64_a"), names
    io = m.conv_io(0)
    assert io.launch == i256[0] + 1          # the conv is complete after the leftover launch
    pre = m.conv_info()[0][0]
    pfx = pre + "." if pre else ""
    w = P[f"{pfx}conv.weight"]
    sc, sh = oracle.bn_fold(P[f"{pfx}bn.weight"], P[f"{pfx}bn.bias"], P[f"{pfx}bn.running_mean"],
                            P[f"{pfx}bn.running_var"], 1e-3)
    xt = to_nhwc(x, vrs.BF16)
    wd, scd, shd = dev(vrs.pack_conv_weight(w, 1, 256, vrs.BF16)), dev(sc), dev(sh)
    y128 = torch.zeros((B, S // 2, S // 2, 256), dtype=torch.bfloat16, device="cuda")
    y256 = torch.zeros_like(y128)
    for yt, tile in ((y128, vrs.TILE_128x128), (y256, vrs.TILE_256x256)):
        ctx().conv2d(vrs.nhwc(xt), wd, scd, shd, vrs.nhwc(yt), 3, 2, 1, vrs.ACT_SILU, None, vrs.BF16, tile=tile)
    torch.cuda.synchronize()
    assert torch.equal(y128.view(torch.int16), y256.view(torch.int16))
    got = out.cpu().numpy().reshape(B, 256, S // 2, S // 2)
    assert np.array_equal(got, from_nhwc(y128, 256, 0))
    ref = oracle.affine_act(oracle.conv2d(x[-2:], w, 2, 1), sc, sh, 1)
    assert rel_err(got[-2:], ref, FLOOR) < TOL


def test_stem_pair_plan():
    """VRS_TILE_STEM_PAIR on model.1: one launch replaces model.0 + model.1,
    bit-identical to the unfused pair on the 128x128 tile (the same MFMA K
    order); conv_io reports the stem as launch-less and model.1 as reading the
    model input (stem = 2).  The entry is refused on any other conv and on a
    width whose stem is not 64 channels (YOLO26n)."""
    import torch
    B, S = 2, 96
    names = [pre for pre, _, _ in _yolo(B, S, vrs.BF16, autotune=False).conv_info()]
    i1 = names.index("model.1")
    plans = {}
    for tile in (vrs.TILE_STEM_PAIR, vrs.TILE_128x128):
        plan = [0] * len(names)
        plan[i1] = tile
        plans[tile] = plan
    x = dev(np.random.default_rng(9).uniform(0, 1, (B, 3, S, S)).astype(np.float32))
    outs = {}
    for tile, plan in plans.items():
        m = _yolo(B, S, vrs.BF16, autotune=False)
        m.set_plan(plan)
        m.load(_params(m))
        outs[tile] = [o.clone() for o in m.forward(x)]
        torch.cuda.synchronize()
        launches = m.launch_names()
        io0, io1 = m.conv_io(names.index("model.0")), m.conv_io(i1)
        if tile == vrs.TILE_STEM_PAIR:
            assert m.get_plan()[i1] == vrs.TILE_STEM_PAIR
            assert io0.launch == -1 and io0.y.data is None
            assert io1.stem == 2 and io1.x.data is None and io1.y.data is not None
            assert launches[io1.launch] == "model.1:vrs_stem_pair_bf16"
            assert not any(l.startswith("model.0:") for l in launches)
        else:
            assert io0.launch >= 0 and io1.stem == 0
    for a, b in zip(outs[vrs.TILE_STEM_PAIR], outs[vrs.TILE_128x128]):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    m = _yolo(1, 128, vrs.BF16, autotune=False)
    bad = [0] * len(names)
    bad[names.index("model.3")] = vrs.TILE_STEM_PAIR
    m.set_plan(bad)
    with pytest.raises(vrs.VrsError):
        m.load(_params(m))
    dn = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="n", one2one=True)
    mn = vrs.Model(ctx(), dn, 1, 128, 128, vrs.BF16, 1e-3, autotune=False)
    names_n = [pre for pre, _, _ in mn.conv_info()]
    bad = [0] * len(names_n)
    bad[names_n.index("model.1")] = vrs.TILE_STEM_PAIR
    mn.set_plan(bad)
    with pytest.raises(vrs.VrsError):
        mn.load(_params(mn))


def test_bottleneck_pair_plan():
    """VRS_TILE_BPAIR on model.2.m.0.cv2 (YOLO26m's 64 -> 32 -> 64 bottleneck
    at stride 4): one launch replaces model.2.m.0.cv1 + cv2, bit-identical to
    both convs on the halo kernel (the same K order and rounding); conv_io
    reports cv1 as launch-less and without output, cv2 as fused_in without
    input.  The entry is refused on a conv that is not a bottleneck's second
    3x3 and on a bottleneck of other widths (YOLO26n's 16 -> 8 -> 16)."""
    import torch
    B, S = 2, 192
    names = [pre for pre, _, _ in _yolo(B, S, vrs.BF16, autotune=False).conv_info()]
    i1, i2 = names.index("model.2.m.0.cv1"), names.index("model.2.m.0.cv2")
    x = dev(np.random.default_rng(5).uniform(0, 1, (B, 3, S, S)).astype(np.float32))
    outs = {}
    for tile in (vrs.TILE_BPAIR, vrs.TILE_H3):
        plan = [0] * len(names)
        plan[i1] = vrs.TILE_H3
        plan[i2] = tile
        m = _yolo(B, S, vrs.BF16, autotune=False)
        m.set_plan(plan)
        m.load(_params(m))
        outs[tile] = [o.clone() for o in m.forward(x)]
        torch.cuda.synchronize()
        launches = m.launch_names()
        io1, io2 = m.conv_io(i1), m.conv_io(i2)
        if tile == vrs.TILE_BPAIR:
            assert m.get_plan()[i2] == vrs.TILE_BPAIR
            assert io1.launch == -1 and io1.y.data is None and io1.x.data is not None
            assert io2.fused_in == 1 and io2.x.data is None and io2.y.data is not None
            assert launches[io2.launch] == "model.2.m.0.cv2:vrs_bpair_bf16_c64_h32_w32"
            assert not any(l.startswith("model.2.m.0.cv1:") for l in launches)
        else:
            assert io1.launch >= 0 and io2.fused_in == 0
    for a, b in zip(outs[vrs.TILE_BPAIR], outs[vrs.TILE_H3]):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    for nm in ("model.2.m.0.cv1", "model.3", "model.6.m.0.m.0.cv2"):
        m = _yolo(1, 128, vrs.BF16, autotune=False)
        bad = [0] * len(names)
        bad[names.index(nm)] = vrs.TILE_BPAIR
        m.set_plan(bad)
        with pytest.raises(vrs.VrsError):
            m.load(_params(m))
    dn = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="n", one2one=True)
    mn = vrs.Model(ctx(), dn, 1, 128, 128, vrs.BF16, 1e-3, autotune=False)
    names_n = [pre for pre, _, _ in mn.conv_info()]
    bad = [0] * len(names_n)
    bad[names_n.index("model.2.m.0.cv2")] = vrs.TILE_BPAIR
    mn.set_plan(bad)
    with pytest.raises(vrs.VrsError):
        mn.load(_params(mn))


def test_head_outputs_on_the_weight_stationary_tile():
    """The Detect head's channel-major float32 output convs (box 64 -> 4,
    class 256 -> 80, plain convs with bias) on the weight-stationary 1x1 tile
    give bit-identical outputs to the 128x128 tile: the same K order and the
    same epilogue arithmetic, one dword store per value."""
    import torch
    x = dev(np.random.default_rng(11).uniform(0, 1, (2, 3, 320, 320)).astype(np.float32))
    m0 = _yolo(2, 320, vrs.BF16, autotune=False)
    P = _params(m0)
    m0.load(P)
    names = [pre for pre, _, _ in m0.conv_info()]
    heads = [i for i, nm in enumerate(names) if nm.startswith("model.23.") and nm.endswith(".2")]
    assert len(heads) == 6, [names[i] for i in heads]
    outs = []
    for tile in (vrs.TILE_128x128, vrs.TILE_W1_128):
        plan = m0.get_plan()
        for i in heads:
            plan[i] = tile
        m = _yolo(2, 320, vrs.BF16, autotune=False)
        m.set_plan(plan)
        m.load(P)
        outs.append([o.clone() for o in m.forward(x)])
        launches = m.launch_names()
        for i in heads:
            got = launches[m.conv_io(i).launch]
            want = "vrs_conv_bf16_128x128_k64_a" if tile == vrs.TILE_128x128 else "vrs_conv1w_bf16_128_c"
            assert got.split(":")[1].startswith(want) and (tile == vrs.TILE_128x128 or got.endswith("_f")), got
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_fused_upsample_on_the_256x256_tile():
    """The neck's fused-upsample 1x1 convs (model.13.cv1, model.16.cv1) on the
    256x256 tile, and model.16.cv1's leftover pixel tiles on the 128x128
    fused-upsample tile (batch 44 at 320: 275 tiles on 256 CUs), give outputs
    bit-identical to the whole convs on the 128x128 tile (the same 64-deep K
    step order)."""
    import torch
    x = dev(np.random.default_rng(12).uniform(0, 1, (44, 3, 320, 320)).astype(np.float32))
    m0 = _yolo(44, 320, vrs.BF16, autotune=False)
    P = _params(m0)
    m0.load(P)
    names = [pre for pre, _, _ in m0.conv_info()]
    ups = [names.index("model.13.cv1"), names.index("model.16.cv1")]
    outs = []
    for tile in (vrs.TILE_128x128, vrs.TILE_256x256):
        plan = m0.get_plan()
        for i in ups:
            plan[i] = tile
        m = _yolo(44, 320, vrs.BF16, autotune=False)
        m.set_plan(plan)
        m.load(P)
        outs.append([o.clone() for o in m.forward(x)])
        if tile == vrs.TILE_256x256:
            launches = m.launch_names()
            k16 = [n for n in launches if n.startswith("model.16.cv1:")]
            assert k16 == ["model.16.cv1:vrs_conv_bf16_256x256_k64_u", "model.16.cv1:vrs_conv_bf16_128x128_k64_u"], k16
            assert "model.13.cv1:vrs_conv_bf16_256x256_k64_u" in launches
        m.close()
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_pointwise_pair_plan():
    """VRS_TILE_PWPAIR on the three Detect class output convs
    (model.23.one2one_cv3.{0,1,2}.2): one launch each replaces the 1x1
    256 -> 256 conv before it and the 256 -> 80 logits conv, bit-identical
    to the two launches (the same K order and rounding) at batch 32, 320x320:
    the P3 pair (800 tiles) on the weight-stationary persistent kernel, P4
    and P5 on the one-group-per-tile kernel, whose 64-pixel tiles of the
    20x20 and 10x10 maps cross image boundaries; conv_io reports the first
    conv as launch-less and without output, the second as fused_in without
    input.  The entry is refused on the box output convs (a 3x3 before them)
    and on YOLO26n (64 -> 80 class channels)."""
    import torch
    B, S = 32, 320
    names = [pre for pre, _, _ in _yolo(B, S, vrs.BF16, autotune=False).conv_info()]
    pairs = [(names.index(f"model.23.one2one_cv3.{i}.1.1"), names.index(f"model.23.one2one_cv3.{i}.2"))
             for i in range(3)]
    x = dev(np.random.default_rng(6).uniform(0, 1, (B, 3, S, S)).astype(np.float32))
    outs = {}
    for tile in (vrs.TILE_PWPAIR, 0):
        plan = [0] * len(names)
        for _, i2 in pairs:
            plan[i2] = tile
        m = _yolo(B, S, vrs.BF16, autotune=False)
        m.set_plan(plan)
        m.load(_params(m))
        outs[tile] = [o.clone() for o in m.forward(x)]
        torch.cuda.synchronize()
        launches = m.launch_names()
        for i1, i2 in pairs:
            io1, io2 = m.conv_io(i1), m.conv_io(i2)
            if tile == vrs.TILE_PWPAIR:
                assert m.get_plan()[i2] == vrs.TILE_PWPAIR
                assert io1.launch == -1 and io1.y.data is None and io1.x.data is not None
                assert io2.fused_in == 1 and io2.x.data is None and io2.out_idx == 1
                kern = "vrs_pwpair_w_bf16_c256_m256" if i2 == pairs[0][1] else "vrs_pwpair_bf16_c256_m256"
                assert launches[io2.launch] == f"{names[i2]}:{kern}"
                assert not any(l.startswith(names[i1] + ":") for l in launches)
            else:
                assert io1.launch >= 0 and io2.fused_in == 0
    for a, b in zip(outs[vrs.TILE_PWPAIR], outs[0]):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    for nm in ("model.23.one2one_cv2.0.2", "model.23.one2one_cv3.0.1.1"):
        m = _yolo(1, 128, vrs.BF16, autotune=False)
        bad = [0] * len(names)
        bad[names.index(nm)] = vrs.TILE_PWPAIR
        m.set_plan(bad)
        with pytest.raises(vrs.VrsError):
            m.load(_params(m))
    dn = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="n", one2one=True)
    mn = vrs.Model(ctx(), dn, 1, 128, 128, vrs.BF16, 1e-3, autotune=False)
    names_n = [pre for pre, _, _ in mn.conv_info()]
    bad = [0] * len(names_n)
    bad[names_n.index("model.23.one2one_cv3.0.2")] = vrs.TILE_PWPAIR
    mn.set_plan(bad)
    with pytest.raises(vrs.VrsError):
        mn.load(_params(mn))
