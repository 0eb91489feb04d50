"""GPU parity of the single-op C-ABI entry points against the CPU oracle.

Inputs and weights are rounded to the kernel's element type first, so the
tolerance measures kernel error, not input quantisation.  Tolerances (from the
north_star): float32 1e-4 relative, bfloat16 2e-2 relative, elementwise, with
an absolute floor for elements near zero (rel_err in gpu_util):
  |got - ref| <= tol * max(|ref|, floor * rms(ref))
floor = 0.05 for float32: two float32 summations of K products differ by
~eps*sqrt(K/2)*rms (~1e-6 rms at K = 576), which the floor must admit;
floor = 0.1 for bfloat16: the attention's probabilities enter the PV MFMA as
bfloat16 (8-bit mantissa), an absolute error of ~2^-9 * rms on every output.
Integer/index/bytes outputs (pooling, upsample, top-k indices) are compared
exactly.
"""
import zlib

import numpy as np
import pytest

import oracle
from gpu_util import bf16_round, ctx, dev, from_nhwc, rel_err, rounder, tdtype, to_nhwc, vrs

pytestmark = pytest.mark.gpu

TOL = {vrs.F32: 1e-4, vrs.BF16: 2e-2}
FLOOR = {vrs.F32: 5e-2, vrs.BF16: 1e-1}
DT = [vrs.F32, vrs.BF16]

CONV_CASES = [
    # n, cin, h, w, cout, k, s, residual, (x pitch, x c_off), (y pitch, y c_off)
    (2, 64, 20, 20, 128, 3, 1, False, None, None),
    (2, 32, 17, 13, 48, 3, 2, False, None, None),
    (1, 8, 32, 32, 16, 3, 2, False, None, None),      # stem-like (padded Cin)
    (2, 48, 9, 9, 80, 1, 1, False, None, None),       # Cin % 32 != 0, Cout 80
    (1, 128, 8, 8, 4, 1, 1, False, None, None),       # Detect box conv width
    (2, 256, 10, 10, 512, 1, 1, True, None, None),    # residual epilogue
    (2, 64, 12, 12, 64, 3, 1, True, (96, 16), (160, 32)),  # channel-slice views
    (1, 512, 6, 7, 256, 3, 2, False, None, None),
]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("case", CONV_CASES)
def test_conv2d(case, dtype):
    import torch
    n, cin, h, w, cout, k, s, with_res, xv, yv = case
    rnd = rounder(dtype)
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    x = rnd(rng.standard_normal((n, cin, h, w)).astype(np.float32))
    wt = rnd((rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32))
    scale = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    ho, wo = (h + 2 * (k // 2) - k) // s + 1, (w + 2 * (k // 2) - k) // s + 1
    res = rnd(rng.standard_normal((n, cout, ho, wo)).astype(np.float32)) if with_res else None
    ref = oracle.affine_act(oracle.conv2d(x, wt, s, k // 2), scale, shift, 1)
    if with_res:
        ref = ref + res
    xp, xo = xv or (cin, 0)
    yp, yo = yv or (cout, 0)
    C = ctx()
    xt = to_nhwc(x, dtype, xp, xo)
    yt = torch.full((n, ho, wo, yp), 7.0, dtype=tdtype(dtype), device="cuda")
    rt = to_nhwc(res, dtype, yp, yo) if with_res else None
    wp = dev(vrs.pack_conv_weight(wt, 1, cin, dtype))
    C.conv2d(vrs.nhwc(xt, cin, xo), wp, dev(scale), dev(shift), vrs.nhwc(yt, cout, yo), k, s, 1, vrs.ACT_SILU,
             vrs.nhwc(rt, cout, yo) if with_res else None, dtype)
    torch.cuda.synchronize()
    got = from_nhwc(yt, cout, yo)
    err = rel_err(got, ref, FLOOR[dtype])
    assert err < TOL[dtype], err
    # channels outside the output view are untouched
    if yp > cout:
        rest = torch.cat([yt[..., :yo], yt[..., yo + cout:]], -1).float()
        assert torch.all(rest == 7.0)


def _random_conv_cases(n_cases, seed):
    """Seeded random dense-conv shapes: ragged pixel and channel counts, both
    kernel sizes and strides, residual on or off, channel-slice input/output
    views, and a tile drawn from those built for the dtype."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n_cases):
        k = int(rng.choice([1, 3]))
        s = int(rng.choice([1, 2])) if k == 3 else 1
        cin = int(rng.choice([8, 16, 24, 32, 40, 64, 96, 128, 192, 256]))
        cout = int(rng.integers(1, 40)) * 8
        n = int(rng.integers(1, 4))
        h, w = int(rng.integers(3, 23)), int(rng.integers(3, 23))
        res = bool(rng.integers(0, 2))
        xo = int(rng.choice([0, 8]))
        yo = int(rng.choice([0, 8, 16]))
        cases.append((n, cin, h, w, cout, k, s, res, xo, yo, int(rng.integers(0, 1 << 30))))
    return cases


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("case", _random_conv_cases(24, 2026))
def test_conv2d_random(case, dtype):
    """24 seeded random shapes per dtype, each on one tile drawn from the
    tiles built for the dtype (the 64-deep step whenever Cin allows it),
    against the oracle; bytes outside the output view stay untouched."""
    import torch
    n, cin, h, w, cout, k, s, with_res, xo, yo, tseed = case
    trng = np.random.default_rng(tseed)
    tiles = TILES_BF16 + [vrs.TILE_256x256] if dtype == vrs.BF16 else TILES_F32
    tile = int(trng.choice(tiles))
    if tile == vrs.TILE_256x256 and cin % 64:
        tile = vrs.TILE_128x128
    if cin % 32 and tile not in (vrs.TILE_128x128, vrs.TILE_64x256, vrs.TILE_32x256):
        tile = vrs.TILE_64x256    # unaligned Cin: the generic-load kernels
    if dtype == vrs.BF16 and trng.integers(0, 2) and tile != vrs.TILE_256x256:
        tile |= vrs.TILE_K32
    rnd = rounder(dtype)
    x = rnd(trng.standard_normal((n, cin, h, w)).astype(np.float32))
    wt = rnd((trng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32))
    scale = trng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = trng.normal(0, 0.2, cout).astype(np.float32)
    ho, wo = (h + 2 * (k // 2) - k) // s + 1, (w + 2 * (k // 2) - k) // s + 1
    ref = oracle.affine_act(oracle.conv2d(x, wt, s, k // 2), scale, shift, 1)
    res = rnd(trng.standard_normal((n, cout, ho, wo)).astype(np.float32)) if with_res else None
    if with_res:
        ref = ref + res
    xp, yp = cin + xo + 8 * (xo > 0), cout + yo + 8
    xt = to_nhwc(x, dtype, xp, xo)
    yt = torch.full((n, ho, wo, yp), 7.0, dtype=tdtype(dtype), device="cuda")
    rt = to_nhwc(res, dtype, yp, yo) if with_res else None
    ctx().conv2d(vrs.nhwc(xt, cin, xo), dev(vrs.pack_conv_weight(wt, 1, cin, dtype)), dev(scale), dev(shift),
                 vrs.nhwc(yt, cout, yo), k, s, 1, vrs.ACT_SILU, vrs.nhwc(rt, cout, yo) if with_res else None, dtype,
                 tile=tile)
    torch.cuda.synchronize()
    assert rel_err(from_nhwc(yt, cout, yo), ref, FLOOR[dtype]) < TOL[dtype], (case, tile)
    rest = torch.cat([yt[..., :yo], yt[..., yo + cout:]], -1).float()
    assert torch.all(rest == 7.0)


TILES_BF16 = [vrs.TILE_128x128, vrs.TILE_256x128, vrs.TILE_128x256, vrs.TILE_64x256, vrs.TILE_32x256,
              vrs.TILE_64x64]
TILES_F32 = [vrs.TILE_128x128, vrs.TILE_64x256, vrs.TILE_32x256]


@pytest.mark.parametrize("dtype,tile", [(vrs.BF16, t) for t in TILES_BF16 + [vrs.TILE_256x256]] +
                         [(vrs.BF16, t | vrs.TILE_K32) for t in TILES_BF16[:4] + [vrs.TILE_64x64]] +
                         [(vrs.F32, t) for t in TILES_F32])
@pytest.mark.parametrize("yview", [(264, 8), (260, 4)])  # staged (16-byte chunks) / direct epilogue
def test_conv2d_every_tile(dtype, tile, yview):
    import torch
    n, cin, h, w, cout, k, s = 2, 128, 14, 10, 256, 3, 1
    rnd = rounder(dtype)
    rng = np.random.default_rng(21)
    x = rnd(rng.standard_normal((n, cin, h, w)).astype(np.float32))
    wt = rnd((rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32))
    scale = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    res = rnd(rng.standard_normal((n, cout, h, w)).astype(np.float32))
    ref = oracle.affine_act(oracle.conv2d(x, wt, s, k // 2), scale, shift, 1) + res
    yp, yo = yview
    xt = to_nhwc(x, dtype)
    yt = torch.full((n, h, w, yp), 7.0, dtype=tdtype(dtype), device="cuda")
    rt = to_nhwc(res, dtype, yp, yo)
    wp = dev(vrs.pack_conv_weight(wt, 1, cin, dtype))
    ctx().conv2d(vrs.nhwc(xt), wp, dev(scale), dev(shift), vrs.nhwc(yt, cout, yo), k, s, 1, vrs.ACT_SILU,
                 vrs.nhwc(rt, cout, yo), dtype, tile=tile)
    torch.cuda.synchronize()
    assert rel_err(from_nhwc(yt, cout, yo), ref, FLOOR[dtype]) < TOL[dtype]
    rest = torch.cat([yt[..., :yo], yt[..., yo + cout:]], -1).float()
    assert torch.all(rest == 7.0)


H3_CASES = [
    # n, cin, h, w, cout, residual, (y pitch, y c_off): strip widths (whole
    # width up to 40, 20 or 32 beyond, partial last strip at 41/70), runs of
    # 256 pixels that start mid-row and end past the image, Cout 32 (narrow
    # kernel) / partial 64-channel tiles, several 32-channel stages
    (2, 64, 160, 160, 32, False, None),
    (1, 32, 80, 80, 64, True, None),
    (2, 128, 20, 20, 128, True, (136, 8)),
    (3, 64, 17, 8, 48, False, None),
    (1, 96, 11, 41, 200, True, None),
    (2, 256, 13, 70, 64, False, (80, 16)),
    (1, 32, 40, 40, 16, True, None),
    (1, 512, 9, 33, 96, False, None),
    (6, 32, 160, 160, 64, True, None),   # 2400 workgroups (residual prefetch across several waves of them)
]


@pytest.mark.parametrize("case", H3_CASES)
def test_conv2d_halo3(case):
    """Halo-tiled 3x3 stride-1 kernel (VRS_TILE_H3) against the oracle, with
    residual and channel-slice output views; bytes outside the view untouched."""
    import torch
    n, cin, h, w, cout, with_res, yv = case
    dtype = vrs.BF16
    rnd = rounder(dtype)
    rng = np.random.default_rng(cin * 7 + cout + h)
    x = rnd(rng.standard_normal((n, cin, h, w)).astype(np.float32))
    wt = rnd((rng.standard_normal((cout, cin, 3, 3)) * np.sqrt(2.0 / (cin * 9))).astype(np.float32))
    scale = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    ref = oracle.affine_act(oracle.conv2d(x, wt, 1, 1), scale, shift, 1)
    res = rnd(rng.standard_normal((n, cout, h, w)).astype(np.float32)) if with_res else None
    if with_res:
        ref = ref + res
    yp, yo = yv or (cout, 0)
    yt = torch.full((n, h, w, yp), 7.0, dtype=torch.bfloat16, device="cuda")
    rt = to_nhwc(res, dtype, yp, yo) if with_res else None
    xt = to_nhwc(x, dtype)   # kept alive until the kernel has run
    ctx().conv2d(vrs.nhwc(xt), dev(vrs.pack_conv_weight(wt, 1, cin, dtype)), dev(scale), dev(shift),
                 vrs.nhwc(yt, cout, yo), 3, 1, 1, vrs.ACT_SILU, vrs.nhwc(rt, cout, yo) if with_res else None, dtype,
                 tile=vrs.TILE_H3)
    torch.cuda.synchronize()
    assert rel_err(from_nhwc(yt, cout, yo), ref, FLOOR[dtype]) < TOL[dtype]
    if yp > cout:
        rest = torch.cat([yt[..., :yo], yt[..., yo + cout:]], -1).float()
        assert torch.all(rest == 7.0)


# (n, h, w, residual, input/output channel layout: (buffer pitch, x offset, y offset) or None)
BPAIR_CASES = [
    (2, 16, 32, True, None),
    (1, 20, 40, True, (192, 64, 128)),   # partial strip and run; C2f-style views of one buffer
    (2, 9, 13, False, None),             # smaller than one run
    (1, 48, 96, True, (128, 0, 64)),
]


@pytest.mark.parametrize("case", BPAIR_CASES)
def test_conv_bottleneck_pair(case):
    """vrs_conv_bottleneck_pair (3x3 64 -> 32 -> 3x3 32 -> 64, SiLU, optional
    residual) equals, bit for bit, the two halo-kernel launches it replaces
    (the middle map written to memory in between), and is within the bf16 bar
    of the oracle bottleneck (the middle map rounded to bf16 where the GPU
    rounds it); bytes outside the output view untouched."""
    import torch
    n, h, w, with_res, lay = case
    C, CH = 64, 32
    rng = np.random.default_rng(h * 31 + w)
    x = bf16_round(rng.standard_normal((n, C, h, w)).astype(np.float32))
    w1 = bf16_round((rng.standard_normal((CH, C, 3, 3)) * np.sqrt(2.0 / (C * 9))).astype(np.float32))
    w2 = bf16_round((rng.standard_normal((C, CH, 3, 3)) * np.sqrt(2.0 / (CH * 9))).astype(np.float32))
    s1, b1 = rng.uniform(0.5, 1.5, CH).astype(np.float32), rng.normal(0, 0.2, CH).astype(np.float32)
    s2, b2 = rng.uniform(0.5, 1.5, C).astype(np.float32), rng.normal(0, 0.2, C).astype(np.float32)
    mid = bf16_round(oracle.affine_act(oracle.conv2d(x, w1, 1, 1), s1, s1 * 0 + b1, 1))
    ref = oracle.affine_act(oracle.conv2d(mid, w2, 1, 1), s2, b2, 1) + (x if with_res else 0)
    pitch, xo, yo = lay or (C, 0, 0)
    if lay:   # input, residual and output as channel slices of one buffer (as in C2f)
        buf = torch.full((n, h, w, pitch), 7.0, dtype=torch.bfloat16, device="cuda")
        buf[..., xo:xo + C] = to_nhwc(x, vrs.BF16)
        xv, yv = vrs.nhwc(buf, C, xo), vrs.nhwc(buf, C, yo)
        outs = [buf]
    else:
        xt = to_nhwc(x, vrs.BF16)
        yt = torch.full((n, h, w, C), 7.0, dtype=torch.bfloat16, device="cuda")
        xv, yv = vrs.nhwc(xt), vrs.nhwc(yt)
        outs = [yt]
    wd1, wd2 = dev(vrs.pack_conv_weight(w1, 1, C, vrs.BF16)), dev(vrs.pack_conv_weight(w2, 1, CH, vrs.BF16))
    ctx().conv_bottleneck_pair(xv, wd1, dev(s1), dev(b1), CH, wd2, dev(s2), dev(b2), yv,
                               res=xv if with_res else None)
    torch.cuda.synchronize()
    fused = outs[0].clone()
    # the same two convs on the halo kernel, the middle map in memory
    mt = torch.zeros((n, h, w, CH), dtype=torch.bfloat16, device="cuda")
    ctx().conv2d(xv, wd1, dev(s1), dev(b1), vrs.nhwc(mt), 3, 1, 1, vrs.ACT_SILU, None, vrs.BF16, tile=vrs.TILE_H3)
    if lay:
        buf[..., yo:yo + C] = 7.0
    else:
        yt.fill_(7.0)
    ctx().conv2d(vrs.nhwc(mt), wd2, dev(s2), dev(b2), yv, 3, 1, 1, vrs.ACT_SILU, xv if with_res else None, vrs.BF16,
                 tile=vrs.TILE_H3)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), outs[0].view(torch.int16)), int((fused != outs[0]).sum())
    got = from_nhwc(fused, C, yo)
    assert rel_err(got, ref, FLOOR[vrs.BF16]) < TOL[vrs.BF16]
    if lay:   # channels outside the output slice (including the input slice) untouched
        keep = [c for c in range(pitch) if not yo <= c < yo + C]
        assert torch.equal(fused[..., keep], outs[0][..., keep])


def test_conv_bottleneck_pair_rejections():
    """Shapes and types the fused pair is not built for: VRS_EUNSUPPORTED."""
    import torch
    for C, CH, dtype in ((64, 64, vrs.BF16), (128, 64, vrs.BF16), (64, 32, vrs.F32)):
        x = torch.zeros((1, 8, 8, C), dtype=tdtype(dtype), device="cuda")
        y = torch.zeros((1, 8, 8, C), dtype=tdtype(dtype), device="cuda")
        w1 = torch.zeros(CH * 9 * C, dtype=tdtype(dtype), device="cuda")
        s = torch.ones(C, device="cuda")
        with pytest.raises(vrs.VrsError) as e:
            ctx().conv_bottleneck_pair(vrs.nhwc(x), w1, s, s, CH, w1, s, s, vrs.nhwc(y), dtype=dtype)
        assert e.value.code == -3, (C, CH, dtype)


@pytest.mark.parametrize("case", [(2, 24, 24, 80, None), (2, 12, 12, 96, (320, 64)), (3, 6, 6, 5, None),
                                  (1, 80, 80, 80, None), (8, 80, 80, 80, None), (9, 61, 61, 96, (264, 8))])
def test_conv_pointwise_pair(case):
    """vrs_conv_pointwise_pair (1x1 256 -> 256 BN + SiLU, then a plain 1x1
    256 -> nc into a channel-major float32 output at y[b*sb + p + co*sc]):
    * against the two convs with the middle map the GPU computes (vrs_conv2d
      of the first conv, bf16): the logits equal a float64 restatement of the
      second conv on that map to float32 summation error over 256 products
      (2e-4 with a floor of 1e-2 rms; measured up to 4.3e-5) -- one value of
      the map rounded differently would move a logit by ~|w2| * 2^-8 |m|,
      ~2e-2 of the floor, so the fused kernel rounds the map exactly as the
      conv kernels do;
    * against the oracle's two convs: within the bf16 bar normwise (the map
      rounded to bf16 on the CPU flips a few values near rounding
      boundaries, so elementwise errors grow with the sample size);
    over pixel tiles that cross image boundaries (HW not a multiple of 64),
    an input that is a channel slice of a wider buffer, nc up to 96, and both
    kernels (one group per tile below two tiles per CU; the weight-stationary
    persistent one above: the last two cases, 800 and 524 tiles, the last
    one ragged); float32 words outside the written slices are untouched."""
    import torch
    n, h, w, nc, lay = case
    C = CM = 256
    rng = np.random.default_rng(h * 7 + nc)
    x = bf16_round(rng.standard_normal((n, C, h, w)).astype(np.float32))
    w1 = bf16_round((rng.standard_normal((CM, C, 1, 1)) * np.sqrt(2.0 / C)).astype(np.float32))
    w2 = bf16_round((rng.standard_normal((nc, CM, 1, 1)) * np.sqrt(1.0 / CM)).astype(np.float32))
    s1, b1 = rng.uniform(0.5, 1.5, CM).astype(np.float32), rng.normal(0, 0.2, CM).astype(np.float32)
    s2, b2 = np.ones(nc, np.float32), rng.normal(0, 0.5, nc).astype(np.float32)
    pitch, xo = lay or (C, 0)
    buf = torch.full((n, h, w, pitch), 3.0, dtype=torch.bfloat16, device="cuda")
    buf[..., xo:xo + C] = to_nhwc(x, vrs.BF16)
    xv = vrs.nhwc(buf, C, xo)
    hw = h * w
    off, sb = 7, nc * hw + 13   # a slice of a wider float32 row per image, as the Detect scales share one
    y = torch.full((n * sb,), -5.0, dtype=torch.float32, device="cuda")
    wd1, wd2 = dev(vrs.pack_conv_weight(w1, 1, C, vrs.BF16)), dev(vrs.pack_conv_weight(w2, 1, CM, vrs.BF16))
    ctx().conv_pointwise_pair(xv, wd1, dev(s1), dev(b1), CM, wd2, dev(s2), dev(b2), nc, y[off:], sb, 1, hw)
    mt = torch.zeros((n, h, w, CM), dtype=torch.bfloat16, device="cuda")
    ctx().conv2d(xv, wd1, dev(s1), dev(b1), vrs.nhwc(mt), 1, 1, 1, vrs.ACT_SILU, None, vrs.BF16)
    torch.cuda.synchronize()
    yh = y.cpu().numpy().reshape(n, sb)
    got = yh[:, off:off + nc * hw].reshape(n, nc, h, w)
    mid_gpu = mt.float().cpu().numpy().astype(np.float64).reshape(n * hw, CM)
    exact = (mid_gpu @ w2.reshape(nc, CM).T.astype(np.float64)) * s2 + b2
    exact = exact.reshape(n, h, w, nc).transpose(0, 3, 1, 2)
    assert rel_err(got, exact, 1e-2) < 2e-4
    mid = bf16_round(oracle.affine_act(oracle.conv2d(x, w1, 1, 0), s1, b1, 1))
    ref = oracle.affine_act(oracle.conv2d(mid, w2, 1, 0), s2, b2, 0)   # [n, nc, h, w]
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < TOL[vrs.BF16]
    untouched = np.concatenate([yh[:, :off].ravel(), yh[:, off + nc * hw:].ravel()])
    assert np.all(untouched == -5.0)


def test_conv_pointwise_pair_rejections():
    """Shapes and types the fused pair is not built for: VRS_EUNSUPPORTED."""
    import torch
    for C, CM, nc in ((128, 256, 80), (256, 128, 80), (256, 256, 97)):
        x = torch.zeros((1, 8, 8, C), dtype=torch.bfloat16, device="cuda")
        w = torch.zeros(256 * 256, dtype=torch.bfloat16, device="cuda")
        s = torch.ones(256, device="cuda")
        y = torch.zeros(nc * 64, device="cuda")
        with pytest.raises(vrs.VrsError) as e:
            ctx().conv_pointwise_pair(vrs.nhwc(x), w, s, s, CM, w, s, s, nc, y, nc * 64, 1, 64)
        assert e.value.code == -3, (C, CM, nc)


def test_conv2d_halo3_rejections():
    import torch
    s = torch.ones(64, device="cuda")
    w = torch.zeros(64 * 9 * 64, dtype=torch.bfloat16, device="cuda")
    for (cin, hw, k, st, dt) in [(48, 16, 3, 1, vrs.BF16), (64, 7, 3, 1, vrs.BF16), (64, 16, 3, 2, vrs.BF16),
                                 (64, 16, 1, 1, vrs.BF16), (64, 16, 3, 1, vrs.F32)]:
        tdt = torch.bfloat16 if dt == vrs.BF16 else torch.float32
        x = torch.zeros((1, hw, hw, cin), dtype=tdt, device="cuda")
        ho = (hw + 2 * (k // 2) - k) // st + 1
        y = torch.zeros((1, ho, ho, 64), dtype=tdt, device="cuda")
        with pytest.raises(vrs.VrsError):
            ctx().conv2d(vrs.nhwc(x), w, s, s, vrs.nhwc(y), k, st, 1, vrs.ACT_SILU, None, dt, tile=vrs.TILE_H3)


W1_CASES = [
    # n, cin, h, w, cout, tile, input view (pitch, c_off), act: several tiles
    # per workgroup (odd and even counts), a ragged last pixel tile, partial
    # channel slices, idle workgroups (fewer tiles than streams), an input
    # channel view, every Cin instance
    (2, 192, 40, 40, 256, vrs.TILE_W1_256, None, vrs.ACT_SILU),
    (3, 128, 33, 17, 200, vrs.TILE_W1_256, None, vrs.ACT_SILU),
    (2, 64, 64, 64, 256, vrs.TILE_W1_256, (128, 32), vrs.ACT_NONE),
    (1, 256, 20, 20, 136, vrs.TILE_W1_128, None, vrs.ACT_SILU),
    (2, 128, 50, 70, 128, vrs.TILE_W1_128, (256, 64), vrs.ACT_SILU),
    (1, 192, 9, 9, 64, vrs.TILE_W1_128, None, vrs.ACT_SILU),
    (64, 128, 40, 40, 128, vrs.TILE_W1_128, None, vrs.ACT_SILU),
    (4, 64, 31, 29, 40, vrs.TILE_W1_128, None, vrs.ACT_SILU),
    # Cin 384: pixel tiles streamed in two 192-channel halves
    (3, 384, 30, 27, 256, vrs.TILE_W1_128, None, vrs.ACT_SILU),
    (2, 384, 17, 13, 136, vrs.TILE_W1_128, (448, 32), vrs.ACT_NONE),
    (1, 384, 5, 5, 128, vrs.TILE_W1_128, None, vrs.ACT_SILU),     # one tile in all
    (16, 384, 40, 40, 512, vrs.TILE_W1_128, None, vrs.ACT_SILU),  # several tiles per workgroup
]


@pytest.mark.parametrize("case", W1_CASES)
def test_conv2d_weight_stationary_1x1(case):
    """Weight-stationary 1x1 kernels against the oracle (a sample of images)
    and against the dense 128x128 kernel (every image), into a channel view
    whose other bytes stay untouched."""
    import torch
    n, cin, h, w, cout, tile, xv, act = case
    dtype = vrs.BF16
    rnd = rounder(dtype)
    rng = np.random.default_rng(cin * 3 + cout + h)
    x = rnd(rng.standard_normal((n, cin, h, w)).astype(np.float32))
    wt = rnd((rng.standard_normal((cout, cin, 1, 1)) * np.sqrt(2.0 / cin)).astype(np.float32))
    scale = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    xp, xo = xv or (cin, 0)
    xt = to_nhwc(x, dtype, xp, xo)
    yp, yo = cout + 16, 8
    yt = torch.full((n, h, w, yp), 7.0, dtype=tdtype(dtype), device="cuda")
    wp = dev(vrs.pack_conv_weight(wt, 1, cin, dtype))
    sd, hd = dev(scale), dev(shift)
    ctx().conv2d(vrs.nhwc(xt, cin, xo), wp, sd, hd, vrs.nhwc(yt, cout, yo), 1, 1, 1, act, None, dtype, tile=tile)
    torch.cuda.synchronize()
    ns = min(n, 2)
    ref = oracle.affine_act(oracle.conv2d(x[:ns], wt, 1, 0), scale, shift, act)
    assert rel_err(from_nhwc(yt[:ns], cout, yo), ref, FLOOR[dtype]) < TOL[dtype]
    y2 = torch.full_like(yt, 7.0)
    ctx().conv2d(vrs.nhwc(xt, cin, xo), wp, sd, hd, vrs.nhwc(y2, cout, yo), 1, 1, 1, act, None, dtype,
                 tile=vrs.TILE_128x128)
    torch.cuda.synchronize()
    assert rel_err(from_nhwc(yt, cout, yo), from_nhwc(y2, cout, yo), FLOOR[dtype]) < TOL[dtype]
    rest = torch.cat([yt[..., :yo], yt[..., yo + cout:]], -1).float()
    assert torch.all(rest == 7.0)


def test_conv2d_weight_stationary_rejections():
    import torch
    s = torch.ones(512, device="cuda")
    w = torch.zeros(512 * 9 * 320, dtype=torch.bfloat16, device="cuda")
    x64 = torch.zeros((1, 8, 8, 64), dtype=torch.bfloat16, device="cuda")
    y64 = torch.zeros((1, 8, 8, 64), dtype=torch.bfloat16, device="cuda")
    for (cin, k, tile) in [(96, 1, vrs.TILE_W1_128), (320, 1, vrs.TILE_W1_128), (256, 1, vrs.TILE_W1_256),
                           (64, 3, vrs.TILE_W1_128)]:
        x = torch.zeros((1, 8, 8, cin), dtype=torch.bfloat16, device="cuda")
        with pytest.raises(vrs.VrsError):
            ctx().conv2d(vrs.nhwc(x), w, s, s, vrs.nhwc(y64), k, 1, 1, vrs.ACT_SILU, None, vrs.BF16, tile=tile)
    with pytest.raises(vrs.VrsError):   # residual
        ctx().conv2d(vrs.nhwc(x64), w, s, s, vrs.nhwc(y64), 1, 1, 1, vrs.ACT_SILU, vrs.nhwc(y64), vrs.BF16,
                     tile=vrs.TILE_W1_128)
    with pytest.raises(vrs.VrsError):   # float32
        xf = torch.zeros((1, 8, 8, 64), dtype=torch.float32, device="cuda")
        ctx().conv2d(vrs.nhwc(xf), w, s, s, vrs.nhwc(xf), 1, 1, 1, vrs.ACT_SILU, None, vrs.F32, tile=vrs.TILE_W1_128)
    with pytest.raises(vrs.VrsError):   # output channel count not a multiple of 8
        y60 = torch.zeros((1, 8, 8, 60), dtype=torch.bfloat16, device="cuda")
        ctx().conv2d(vrs.nhwc(x64), w, s, s, vrs.nhwc(y60), 1, 1, 1, vrs.ACT_SILU, None, vrs.BF16,
                     tile=vrs.TILE_W1_128)


PERSIST_CASES = [
    # n, cin, h, w, cout, k, s, tile: several tiles per workgroup, ragged pixel
    # and channel tiles, padding taps, stride 2, both step depths
    (8, 128, 96, 96, 256, 1, 1, vrs.TILE_128x128 | vrs.TILE_K32 | vrs.TILE_PERSIST),
    (8, 128, 96, 96, 256, 1, 1, vrs.TILE_128x128 | vrs.TILE_PERSIST),
    (3, 192, 50, 70, 80, 1, 1, vrs.TILE_128x128 | vrs.TILE_K32 | vrs.TILE_PERSIST),
    (4, 64, 60, 60, 64, 3, 1, vrs.TILE_64x256 | vrs.TILE_K32 | vrs.TILE_PERSIST),
    (2, 64, 41, 37, 32, 3, 2, vrs.TILE_64x256 | vrs.TILE_K32 | vrs.TILE_PERSIST),
    (2, 128, 30, 22, 128, 3, 1, vrs.TILE_128x128 | vrs.TILE_PERSIST),
    # 256x256 (8 waves, epilogue stored from the accumulators): 966 tiles on
    # 256 workgroups (3-4 each); 576 tiles = 2 rounds + 64 leftover tiles on
    # the 128x128 tile; a 3x3/s2 conv with 273 tiles (1 round + 17 leftover)
    (16, 128, 112, 138, 256, 1, 1, vrs.TILE_256x256 | vrs.TILE_PERSIST),
    (16, 128, 96, 96, 256, 1, 1, vrs.TILE_256x256 | vrs.TILE_PERSIST),
    (64, 128, 66, 66, 256, 3, 2, vrs.TILE_256x256 | vrs.TILE_PERSIST),
]


@pytest.mark.parametrize("case", PERSIST_CASES)
def test_conv2d_persistent(case):
    """Persistent-grid conv (one load stream across a workgroup's tiles) into a
    channel view, against the oracle; bytes outside the view stay untouched."""
    import torch
    n, cin, h, w, cout, k, s, tile = case
    dtype = vrs.BF16
    rnd = rounder(dtype)
    rng = np.random.default_rng(cin + cout + k)
    x = rnd(rng.standard_normal((n, cin, h, w)).astype(np.float32))
    wt = rnd((rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32))
    scale = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    xt = to_nhwc(x, dtype)
    ho, wo = (h + 2 * (k // 2) - k) // s + 1, (w + 2 * (k // 2) - k) // s + 1
    yp, yo = cout + 16, 8
    yt = torch.full((n, ho, wo, yp), 7.0, dtype=tdtype(dtype), device="cuda")
    wp = dev(vrs.pack_conv_weight(wt, 1, cin, dtype))
    ctx().conv2d(vrs.nhwc(xt), wp, dev(scale), dev(shift), vrs.nhwc(yt, cout, yo), k, s, 1, vrs.ACT_SILU, None,
                 dtype, tile=tile)
    torch.cuda.synchronize()
    # the oracle on a sample of images keeps the check fast at these sizes
    ns = min(n, 2)
    ref = oracle.affine_act(oracle.conv2d(x[:ns], wt, s, k // 2), scale, shift, 1)
    assert rel_err(from_nhwc(yt[:ns], cout, yo), ref, FLOOR[dtype]) < TOL[dtype]
    # every image: same result as the non-persistent kernel of the same tile
    y2 = torch.full_like(yt, 7.0)
    ctx().conv2d(vrs.nhwc(xt), wp, dev(scale), dev(shift), vrs.nhwc(y2, cout, yo), k, s, 1, vrs.ACT_SILU, None,
                 dtype, tile=tile & ~vrs.TILE_PERSIST)
    torch.cuda.synchronize()
    assert torch.equal(yt, y2)


def test_conv2d_persistent_rejections():
    import torch
    t = vrs.TILE_128x128 | vrs.TILE_K32 | vrs.TILE_PERSIST
    x = torch.zeros((1, 8, 8, 96), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((1, 8, 8, 128), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(128 * 96, dtype=torch.bfloat16, device="cuda")
    s = torch.ones(128, device="cuda")
    with pytest.raises(vrs.VrsError):   # 3 K steps: odd
        ctx().conv2d(vrs.nhwc(x), w, s, s, vrs.nhwc(y), 1, 1, 1, vrs.ACT_SILU, None, vrs.BF16, tile=t)
    x = torch.zeros((1, 8, 8, 128), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(128 * 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(vrs.VrsError):   # residual
        ctx().conv2d(vrs.nhwc(x), w, s, s, vrs.nhwc(y), 1, 1, 1, vrs.ACT_SILU, vrs.nhwc(y), vrs.BF16, tile=t)
    with pytest.raises(vrs.VrsError):   # float32
        ctx().conv2d(vrs.nhwc(x.float()), w, s, s, vrs.nhwc(y.float()), 1, 1, 1, vrs.ACT_SILU, None, vrs.F32,
                     tile=t)


FP8_CASES = [
    # n, cin, h, w, cout, k, s, residual, tile
    (2, 64, 20, 20, 128, 3, 1, False, vrs.TILE_128x128),
    (2, 128, 9, 11, 256, 3, 2, False, vrs.TILE_256x128),
    (2, 192, 12, 12, 64, 1, 1, True, vrs.TILE_64x256),
    (1, 256, 10, 10, 96, 3, 1, False, vrs.TILE_128x256),
    (2, 64, 15, 7, 200, 1, 1, True, vrs.TILE_AUTO),
    (2, 128, 14, 10, 256, 3, 1, True, vrs.TILE_256x256),
    (1, 256, 9, 13, 320, 3, 2, False, vrs.TILE_256x256),
]


@pytest.mark.parametrize("case", FP8_CASES)
def test_conv2d_fp8(case):
    """e4m3 weights (per-channel absmax/448) and e4m3-quantised bf16 inputs
    (power-of-two step) on the fp8 MFMA, against the oracle conv of the same
    dequantised operands: only accumulation order and the bf16 output
    rounding differ, so the bf16 bar applies."""
    import torch
    n, cin, h, w, cout, k, s, with_res, tile = case
    rng = np.random.default_rng(31 + cin)
    x = bf16_round(rng.standard_normal((n, cin, h, w)).astype(np.float32) * 3.0)
    wt = (rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)
    bn_s = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    in_scale = float(2.0 ** np.ceil(np.log2(np.abs(x).max() / 448.0)))
    q, ws = vrs.pack_conv_weight_fp8(wt)
    from oracle.yolo26 import fp8_conv_inputs
    xq, wq = fp8_conv_inputs(x, wt, in_scale)
    ho, wo = (h + 2 * (k // 2) - k) // s + 1, (w + 2 * (k // 2) - k) // s + 1
    res = bf16_round(rng.standard_normal((n, cout, ho, wo)).astype(np.float32)) if with_res else None
    ref = oracle.affine_act(oracle.conv2d(xq, wq, s, k // 2), bn_s, shift, 1)
    if with_res:
        ref = ref + res
    xt = to_nhwc(x, vrs.BF16)
    yt = torch.full((n, ho, wo, cout), 7.0, dtype=torch.bfloat16, device="cuda")
    rt = to_nhwc(res, vrs.BF16) if with_res else None
    ctx().conv2d(vrs.nhwc(xt), dev(q), dev((bn_s * ws * in_scale).astype(np.float32)), dev(shift), vrs.nhwc(yt),
                 k, s, 1, vrs.ACT_SILU, vrs.nhwc(rt) if with_res else None, vrs.FP8, tile=tile, in_scale=in_scale)
    torch.cuda.synchronize()
    assert rel_err(from_nhwc(yt), ref, FLOOR[vrs.BF16]) < TOL[vrs.BF16]


@pytest.mark.parametrize("case", [(2, 128, 12, 10, 128, 2, 3, 1, True), (1, 256, 9, 9, 192, 2, 1, 1, False)])
def test_grouped_conv2d_fp8(case):
    """Grouped conv on the fp8 route (one e4m3 implicit-GEMM launch per group,
    weights from pack_conv_weight_fp8 over Cin/groups inputs) against the
    oracle's grouped conv of the same dequantised operands; Cin/groups not a
    multiple of 64 is refused."""
    import torch
    n, cin, h, w, cout, G, k, s, with_res = case
    rng = np.random.default_rng(41 + cin)
    x = bf16_round(rng.standard_normal((n, cin, h, w)).astype(np.float32) * 3.0)
    wt = (rng.standard_normal((cout, cin // G, k, k)) * np.sqrt(2.0 / (cin // G * k * k))).astype(np.float32)
    bn_s = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    in_scale = float(2.0 ** np.ceil(np.log2(np.abs(x).max() / 448.0)))
    q, ws = vrs.pack_conv_weight_fp8(wt)
    from oracle.yolo26 import fp8_conv_inputs
    xq, wq = fp8_conv_inputs(x, wt, in_scale)
    ho, wo = (h + 2 * (k // 2) - k) // s + 1, (w + 2 * (k // 2) - k) // s + 1
    res = bf16_round(rng.standard_normal((n, cout, ho, wo)).astype(np.float32)) if with_res else None
    ref = oracle.affine_act(oracle.conv2d(xq, wq, s, k // 2, groups=G), bn_s, shift, 1)
    if with_res:
        ref = ref + res
    xt = to_nhwc(x, vrs.BF16)
    yt = torch.full((n, ho, wo, cout), 7.0, dtype=torch.bfloat16, device="cuda")
    rt = to_nhwc(res, vrs.BF16) if with_res else None
    sc = dev((bn_s * ws * in_scale).astype(np.float32))
    ctx().conv2d(vrs.nhwc(xt), dev(q), sc, dev(shift), vrs.nhwc(yt), k, s, G, vrs.ACT_SILU,
                 vrs.nhwc(rt) if with_res else None, vrs.FP8, in_scale=in_scale)
    torch.cuda.synchronize()
    assert rel_err(from_nhwc(yt), ref, FLOOR[vrs.BF16]) < TOL[vrs.BF16]
    with pytest.raises(vrs.VrsError) as e:   # 4 groups: 32 (or 64 for Cin 256) inputs each
        ctx().conv2d(vrs.nhwc(xt), dev(q), sc, dev(shift), vrs.nhwc(yt), k, s, 2 * G if cin == 128 else 8,
                     vrs.ACT_SILU, None, vrs.FP8, in_scale=in_scale)
    assert e.value.code == -3


def _e4m3_nhwc(a_nchw, step, pitch=None, c_off=0):
    """NCHW float32 -> device uint8 [n, h, w, pitch] holding e4m3(a / step)
    (round to nearest even, torch.float8_e4m3fn) in channels [c_off, c_off+c),
    and the dequantised values it holds."""
    import torch
    n, c, h, w = a_nchw.shape
    pitch = c if pitch is None else pitch
    q = torch.from_numpy(np.ascontiguousarray(a_nchw.transpose(0, 2, 3, 1)) / np.float32(step)).to(
        torch.float8_e4m3fn)
    t = torch.zeros((n, h, w, pitch), dtype=torch.uint8, device="cuda")
    t[..., c_off:c_off + c] = q.view(torch.uint8).to("cuda")
    return t, (q.float().numpy() * np.float32(step)).transpose(0, 3, 1, 2).copy()


def _from_e4m3_nhwc(t, step, c, c_off=0):
    import torch
    return (t[..., c_off:c_off + c].cpu().view(torch.float8_e4m3fn).float().numpy() * np.float32(step)).transpose(
        0, 3, 1, 2)


def e4m3_bracket(ref, step, tol=TOL[vrs.BF16], floor_frac=FLOOR[vrs.BF16]):
    """The e4m3 outputs an fp8 conv may store for reference values ref: the
    e4m3 rounding (on step, of the bfloat16 value) of something within the
    single-kernel bar of ref, i.e. [Q(ref - t), Q(ref + t)] with
    t = tol * max(|ref|, floor_frac * rms(ref)); Q is monotone."""
    from oracle.yolo26 import e4m3_round
    rms = float(np.sqrt(np.mean(np.asarray(ref, np.float64) ** 2)))
    t = tol * np.maximum(np.abs(ref), floor_frac * rms)
    q = lambda v: e4m3_round(bf16_round(np.asarray(v, np.float32)) / np.float32(step)) * np.float32(step)  # noqa: E731
    return q(ref - t), q(ref + t)


# (n, cin, h, w, cout, k, stride, residual, tile, e4m3 input, e4m3 output, e4m3 residual, channel offset)
FP8_E4M3_CASES = [
    (2, 64, 20, 18, 128, 3, 1, True, vrs.TILE_128x128, True, True, True, 16),
    (2, 128, 16, 16, 64, 1, 1, False, vrs.TILE_64x256, True, True, False, 0),
    (1, 128, 24, 20, 256, 3, 2, False, vrs.TILE_256x128, True, False, False, 32),
    (1, 192, 12, 12, 128, 1, 1, True, vrs.TILE_128x256, False, True, True, 0),
    (1, 256, 20, 20, 256, 3, 2, False, vrs.TILE_256x256, True, True, False, 0),
    (2, 64, 10, 14, 256, 3, 1, True, vrs.TILE_256x256, True, True, True, 64),
    (1, 128, 30, 30, 128, 3, 1, True, vrs.TILE_128x128, False, False, True, 0),
]


@pytest.mark.parametrize("case", FP8_E4M3_CASES)
def test_conv2d_fp8_e4m3_activations(case):
    """fp8 conv with e4m3 activations in memory: an e4m3 input on its step
    (staged into LDS as read), an e4m3 output (the e4m3 rounding, on its
    step, of the bf16 result) and an e4m3 residual, each alone and together,
    on every fp8 tile, in views with a channel offset.  Against the oracle conv
    of the same dequantised operands: a bf16 output to the bf16 bar, an e4m3
    output inside the e4m3 bracket of that bar (e4m3_bracket)."""
    import torch
    n, cin, h, w, cout, k, s, with_res, tile, x8, y8, r8, off = case
    rng = np.random.default_rng(71 + cin + cout)
    x = bf16_round(rng.standard_normal((n, cin, h, w)).astype(np.float32) * 2.0)
    wt = (rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)
    bn_s = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    in_scale = float(2.0 ** np.ceil(np.log2(np.abs(x).max() / 448.0)))
    q, ws = vrs.pack_conv_weight_fp8(wt)
    from oracle.yolo26 import fp8_conv_inputs
    xq, wq = fp8_conv_inputs(x, wt, in_scale)
    ho, wo = (h + 2 * (k // 2) - k) // s + 1, (w + 2 * (k // 2) - k) // s + 1
    res = bf16_round(rng.standard_normal((n, cout, ho, wo)).astype(np.float32)) if with_res else None
    res_step = 2.0 ** -5
    if x8:
        xt, xq2 = _e4m3_nhwc(x, in_scale, cin + off, off)
        assert np.array_equal(xq2, xq)
    else:
        xt = to_nhwc(x, vrs.BF16, cin + off, off)
    rt = None
    if with_res:
        if r8:
            rt, res = _e4m3_nhwc(res, res_step, cout + off, off)
        else:
            rt = to_nhwc(res, vrs.BF16, cout + off, off)
    ref = oracle.affine_act(oracle.conv2d(xq, wq, s, k // 2), bn_s, shift, 1)
    if with_res:
        ref = ref + res
    out_step = float(2.0 ** np.ceil(np.log2(np.abs(ref).max() / 448.0)))
    if y8:
        yt = torch.full((n, ho, wo, cout + off), 0x55, dtype=torch.uint8, device="cuda")
    else:
        yt = torch.full((n, ho, wo, cout + off), 7.0, dtype=torch.bfloat16, device="cuda")
    ctx().conv2d(vrs.nhwc(xt, cin, off), dev(q), dev((bn_s * ws * in_scale).astype(np.float32)), dev(shift),
                 vrs.nhwc(yt, cout, off), k, s, 1, vrs.ACT_SILU, vrs.nhwc(rt, cout, off) if with_res else None,
                 vrs.FP8, tile=tile, in_scale=in_scale, x_e4m3=x8, y_e4m3=y8, out_step=out_step if y8 else 0.0,
                 res_e4m3=r8 and with_res, res_step=res_step if (r8 and with_res) else 0.0)
    torch.cuda.synchronize()
    if y8:
        got = _from_e4m3_nhwc(yt, out_step, cout, off)
        lo, hi = e4m3_bracket(ref, out_step)
        bad = (got < lo) | (got > hi)
        assert not bad.any(), (int(bad.sum()), got[bad][:4], ref[bad][:4])
        assert torch.all(yt[..., :off] == 0x55)   # channels before the view untouched
    else:
        assert rel_err(from_nhwc(yt, cout, off), ref, FLOOR[vrs.BF16]) < TOL[vrs.BF16]


# (n, cin, h, w, cout, e4m3 input, e4m3 output, channel offset, act)
FP8_W1_CASES = [
    (2, 128, 20, 18, 128, False, False, 0, vrs.ACT_SILU),
    (1, 192, 16, 16, 256, False, True, 0, vrs.ACT_SILU),
    (2, 256, 12, 11, 64, True, True, 16, vrs.ACT_SILU),
    (1, 256, 9, 7, 128, False, False, 8, vrs.ACT_NONE),
    (1, 384, 10, 13, 512, True, True, 0, vrs.ACT_SILU),
    (1, 512, 9, 9, 192, True, False, 0, vrs.ACT_SILU),
    (1, 512, 7, 9, 256, False, False, 0, vrs.ACT_SILU),
    (1, 768, 8, 10, 512, True, True, 32, vrs.ACT_SILU),
    (1, 768, 12, 12, 256, False, True, 0, vrs.ACT_NONE),
]


@pytest.mark.parametrize("case", FP8_W1_CASES)
def test_conv2d_fp8_weight_stationary(case):
    """The fp8 weight-stationary 1x1 kernel (VRS_TILE_W1_128 on VRS_FP8) on
    every input width it is built for, with bf16 or e4m3 inputs and outputs,
    ragged pixel counts, Cout below and above one 128-channel slice and channel
    offsets: bit-identical to the tiled fp8 kernel (same e4m3 staging, k slices
    in the same order, same output rounding), whose results the other fp8
    tests hold to the oracle; and, on its own, within the bar of the oracle
    conv of the same dequantised operands."""
    import torch
    n, cin, h, w, cout, x8, y8, off, act = case
    rng = np.random.default_rng(91 + cin + cout)
    x = bf16_round(rng.standard_normal((n, cin, h, w)).astype(np.float32) * 2.0)
    wt = (rng.standard_normal((cout, cin, 1, 1)) * np.sqrt(2.0 / cin)).astype(np.float32)
    bn_s = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    in_scale = float(2.0 ** np.ceil(np.log2(np.abs(x).max() / 448.0)))
    q, ws = vrs.pack_conv_weight_fp8(wt)
    from oracle.yolo26 import fp8_conv_inputs
    xq, wq = fp8_conv_inputs(x, wt, in_scale)
    if x8:
        xt, _ = _e4m3_nhwc(x, in_scale, cin + off, off)
    else:
        xt = to_nhwc(x, vrs.BF16, cin + off, off)
    ref = oracle.affine_act(oracle.conv2d(xq, wq, 1, 0), bn_s, shift, act)
    out_step = float(2.0 ** np.ceil(np.log2(np.abs(ref).max() / 448.0)))
    outs = {}
    for tile in (vrs.TILE_128x128, vrs.TILE_W1_128):
        if y8:
            yt = torch.full((n, h, w, cout + off), 0x55, dtype=torch.uint8, device="cuda")
        else:
            yt = torch.full((n, h, w, cout + off), 7.0, dtype=torch.bfloat16, device="cuda")
        ctx().conv2d(vrs.nhwc(xt, cin, off), dev(q), dev((bn_s * ws * in_scale).astype(np.float32)), dev(shift),
                     vrs.nhwc(yt, cout, off), 1, 1, 1, act, None, vrs.FP8, tile=tile, in_scale=in_scale, x_e4m3=x8,
                     y_e4m3=y8, out_step=out_step if y8 else 0.0)
        torch.cuda.synchronize()
        outs[tile] = yt
    a, b = outs[vrs.TILE_128x128], outs[vrs.TILE_W1_128]
    if y8:
        assert torch.equal(a, b), int((a != b).sum())
        got = _from_e4m3_nhwc(b, out_step, cout, off)
        lo, hi = e4m3_bracket(ref, out_step)
        assert not ((got < lo) | (got > hi)).any()
    else:
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), int((a != b).sum())
        assert rel_err(from_nhwc(b, cout, off), ref, FLOOR[vrs.BF16]) < TOL[vrs.BF16]


def test_conv2d_fp8_weight_stationary_rejections():
    """Shapes the fp8 weight-stationary kernel is not built for fail to prepare
    with VRS_EUNSUPPORTED (the autotuner then skips it)."""
    import torch
    sc = torch.ones(128, device="cuda")
    for cin, k, with_res in ((64, 1, False), (320, 1, False), (128, 3, False), (128, 1, True)):
        x = torch.zeros((1, 8, 8, cin), dtype=torch.bfloat16, device="cuda")
        y = torch.zeros((1, 8, 8, 128), dtype=torch.bfloat16, device="cuda")
        w = torch.zeros(128 * cin * k * k, dtype=torch.uint8, device="cuda")
        with pytest.raises(vrs.VrsError) as e:
            ctx().conv2d(vrs.nhwc(x), w, sc, sc, vrs.nhwc(y), k, 1, 1, vrs.ACT_NONE,
                         vrs.nhwc(y) if with_res else None, vrs.FP8, tile=vrs.TILE_W1_128, in_scale=1.0)
        assert e.value.code == -3, (cin, k, with_res)


# (n, cin, h, w, cout, k, stride)
FP8_K128_CASES = [(1, 256, 20, 20, 256, 3, 2), (2, 128, 10, 12, 512, 3, 1), (1, 384, 9, 11, 256, 1, 1)]


@pytest.mark.parametrize("case", FP8_K128_CASES)
def test_conv2d_fp8_k128(case):
    """128-deep K steps on the fp8 256x256 tile (VRS_TILE_K128, e4m3 input):
    within the bar of the oracle conv of the same dequantised operands, and on
    a 1x1 conv (where the 64- and 128-deep orders visit the channels alike)
    bit-identical to the 64-deep tile; a bf16 input is refused."""
    import torch
    n, cin, h, w, cout, k, s = case
    rng = np.random.default_rng(13 + cin + cout)
    x = bf16_round(rng.standard_normal((n, cin, h, w)).astype(np.float32) * 2.0)
    wt = (rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)
    bn_s = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    in_scale = float(2.0 ** np.ceil(np.log2(np.abs(x).max() / 448.0)))
    q, ws = vrs.pack_conv_weight_fp8(wt)
    from oracle.yolo26 import fp8_conv_inputs
    xq, wq = fp8_conv_inputs(x, wt, in_scale)
    xt, _ = _e4m3_nhwc(x, in_scale)
    ho, wo = (h + 2 * (k // 2) - k) // s + 1, (w + 2 * (k // 2) - k) // s + 1
    ref = oracle.affine_act(oracle.conv2d(xq, wq, s, k // 2), bn_s, shift, 1)
    outs = {}
    for tile in (vrs.TILE_256x256, vrs.TILE_256x256 | vrs.TILE_K128):
        yt = torch.full((n, ho, wo, cout), 7.0, dtype=torch.bfloat16, device="cuda")
        ctx().conv2d(vrs.nhwc(xt), dev(q), dev((bn_s * ws * in_scale).astype(np.float32)), dev(shift), vrs.nhwc(yt),
                     k, s, 1, vrs.ACT_SILU, None, vrs.FP8, tile=tile, in_scale=in_scale, x_e4m3=True)
        torch.cuda.synchronize()
        outs[tile] = yt
        assert rel_err(from_nhwc(yt), ref, FLOOR[vrs.BF16]) < TOL[vrs.BF16], hex(tile)
    if k == 1:
        a, b = outs.values()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    xb = to_nhwc(x, vrs.BF16)
    with pytest.raises(vrs.VrsError) as e:
        ctx().conv2d(vrs.nhwc(xb), dev(q), dev(bn_s), dev(shift), vrs.nhwc(outs[vrs.TILE_256x256]), k, s, 1,
                     vrs.ACT_SILU, None, vrs.FP8, tile=vrs.TILE_256x256 | vrs.TILE_K128, in_scale=in_scale)
    assert e.value.code == -3


def test_conv2d_fp8_e4m3_rejections():
    import torch
    x = torch.zeros((1, 4, 4, 72), dtype=torch.uint8, device="cuda")
    y = torch.zeros((1, 4, 4, 64), dtype=torch.uint8, device="cuda")
    w = torch.zeros(64 * 64, dtype=torch.uint8, device="cuda")
    sc = torch.ones(64, device="cuda")
    with pytest.raises(vrs.VrsError):   # e4m3 input view not 16-channel aligned
        ctx().conv2d(vrs.nhwc(x, 64, 8), w, sc, sc, vrs.nhwc(y), 1, 1, 1, vrs.ACT_NONE, None, vrs.FP8,
                     in_scale=1.0, x_e4m3=True)
    x = torch.zeros((1, 4, 4, 64), dtype=torch.uint8, device="cuda")
    with pytest.raises(vrs.VrsError):   # output step not a power of two
        ctx().conv2d(vrs.nhwc(x), w, sc, sc, vrs.nhwc(y), 1, 1, 1, vrs.ACT_NONE, None, vrs.FP8, in_scale=1.0,
                     x_e4m3=True, y_e4m3=True, out_step=0.3)
    y2 = torch.zeros((1, 4, 4, 72), dtype=torch.uint8, device="cuda")
    with pytest.raises(vrs.VrsError):   # e4m3 output view not 16-channel aligned
        ctx().conv2d(vrs.nhwc(x), w, sc, sc, vrs.nhwc(y2, 64, 8), 1, 1, 1, vrs.ACT_NONE, None, vrs.FP8,
                     in_scale=1.0, x_e4m3=True, y_e4m3=True, out_step=1.0)
    xb = torch.zeros((1, 4, 4, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(vrs.VrsError):   # e4m3 activations on a bf16 conv
        ctx().conv2d(vrs.nhwc(xb), w, sc, sc, vrs.nhwc(y), 1, 1, 1, vrs.ACT_NONE, None, vrs.BF16,
                     x_e4m3=True)


def test_conv2d_fp8_rejections():
    import torch
    x = torch.zeros((1, 4, 4, 32), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((1, 4, 4, 64), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(64 * 32, dtype=torch.uint8, device="cuda")
    sc = torch.ones(64, device="cuda")
    with pytest.raises(vrs.VrsError):   # Cin % 64 != 0
        ctx().conv2d(vrs.nhwc(x), w, sc, sc, vrs.nhwc(y), 1, 1, 1, vrs.ACT_NONE, None, vrs.FP8, in_scale=1.0)
    x = torch.zeros((1, 4, 4, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(vrs.VrsError):   # step not a power of two
        ctx().conv2d(vrs.nhwc(x), w, sc, sc, vrs.nhwc(y), 1, 1, 1, vrs.ACT_NONE, None, vrs.FP8, in_scale=0.3)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("shape", [(2, 64, 40, 66), (1, 16, 18, 30), (1, 96, 10, 128), (1, 64, 640, 640),
                                   (1, 32, 7, 9), (1, 128, 12, 20), (3, 40, 130, 132)])
def test_conv_stem(dtype, shape):
    """Fused stem (NCHW float32 image -> NHWC, 3x3 s2) against the oracle conv."""
    import torch
    n, cout, h, w = shape
    rnd = rounder(dtype)
    rng = np.random.default_rng(11 + cout)
    x = rnd(rng.uniform(0, 1, (n, 3, h, w)).astype(np.float32))
    wt = rnd((rng.standard_normal((cout, 3, 3, 3)) * np.sqrt(2.0 / 27)).astype(np.float32))
    scale = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    ref = oracle.affine_act(oracle.conv2d(x, wt, 2, 1), scale, shift, 1)
    ho, wo = ref.shape[2], ref.shape[3]
    yt = torch.full((n, ho, wo, cout + 16), 7.0, dtype=tdtype(dtype), device="cuda")
    ctx().conv_stem(dev(x), dev(vrs.pack_stem_weight(wt, dtype)), dev(scale), dev(shift), vrs.nhwc(yt, cout, 8),
                    vrs.ACT_SILU, dtype)
    torch.cuda.synchronize()
    assert rel_err(from_nhwc(yt, cout, 8), ref, FLOOR[dtype]) < TOL[dtype]
    rest = torch.cat([yt[..., :8], yt[..., 8 + cout:]], -1).float()
    assert torch.all(rest == 7.0)


def test_conv2d_tile_rejections():
    import torch
    x = torch.zeros((1, 4, 4, 48), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((1, 4, 4, 64), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(64 * 48, dtype=torch.bfloat16, device="cuda")
    s = torch.ones(64, device="cuda")
    with pytest.raises(vrs.VrsError):  # 256x128 needs Cin % 32 == 0
        ctx().conv2d(vrs.nhwc(x), w, s, s, vrs.nhwc(y), 1, 1, 1, vrs.ACT_SILU, None, vrs.BF16, tile=vrs.TILE_256x128)
    with pytest.raises(vrs.VrsError):  # no float32 build of 128x256
        ctx().conv2d(vrs.nhwc(x.float()), w, s, s, vrs.nhwc(y.float()), 1, 1, 1, vrs.ACT_SILU, None, vrs.F32,
                     tile=vrs.TILE_128x256)


DW_SHAPES = [
    # n, c, h, w, strides: band/patch/channel-block edges of the row-walking
    # stride-1 kernel (bands of 10 rows below 32 rows, 40 from there on;
    # 8-column patches; 64-channel blocks) and the generic stride-2 kernel
    (2, 64, 11, 9, (1, 2)),
    (1, 200, 70, 20, (1,)),
    (2, 72, 40, 12, (1,)),      # one whole 40-row band
    (1, 64, 83, 9, (1,)),       # two whole bands and a 3-row one
    (2, 24, 3, 3, (1, 2)),
    (1, 136, 21, 17, (1,)),
]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("act", [vrs.ACT_SILU, vrs.ACT_NONE])
@pytest.mark.parametrize("shape", DW_SHAPES)
def test_dwconv(dtype, act, shape):
    import torch
    rnd = rounder(dtype)
    rng = np.random.default_rng(7)
    n, c, h, w, strides = shape
    x = rnd(rng.standard_normal((n, c, h, w)).astype(np.float32))
    wt = rnd((rng.standard_normal((c, 1, 3, 3)) * 0.4).astype(np.float32))
    scale = rng.uniform(0.5, 1.5, c).astype(np.float32)
    shift = rng.normal(0, 0.2, c).astype(np.float32)
    C = ctx()
    xt = to_nhwc(x, dtype, c + 32, 8)
    for s in strides:
        ref = oracle.affine_act(oracle.conv2d(x, wt, s, 1, groups=c), scale, shift, act)
        yt = torch.full((n, ref.shape[2], ref.shape[3], c + 16), 7.0, dtype=tdtype(dtype), device="cuda")
        C.conv2d(vrs.nhwc(xt, c, 8), dev(vrs.pack_conv_weight(wt, c, 1, dtype)), dev(scale), dev(shift),
                 vrs.nhwc(yt, c, 8), 3, s, c, act, None, dtype)
        torch.cuda.synchronize()
        assert rel_err(from_nhwc(yt, c, 8), ref, FLOOR[dtype]) < TOL[dtype], s
        rest = torch.cat([yt[..., :8], yt[..., 8 + c:]], -1).float()
        assert torch.all(rest == 7.0)


GCONV_CASES = [
    # n, cin, h, w, cout, groups, k, s, residual, (x pitch, x c_off), (y pitch, y c_off)
    (2, 8, 9, 7, 12, 4, 3, 1, False, None, None),              # direct kernel: 2 -> 3 channels per group
    (2, 24, 10, 11, 36, 3, 3, 2, True, (40, 5), (48, 3)),      # direct: odd channel offsets, residual
    (1, 6, 5, 5, 4, 2, 1, 1, False, None, None),               # direct, 1x1
    (2, 64, 7, 6, 64, 8, 5, 1, False, None, None),             # direct, 5x5, 8 x 8 per group
    (2, 128, 12, 12, 128, 2, 3, 1, True, None, None),          # one dense launch per group (64 x 64)
    (2, 256, 9, 9, 128, 4, 1, 1, False, (272, 16), (144, 8)),  # dense per group on channel slices
    (1, 96, 11, 13, 192, 3, 3, 2, False, None, None),          # dense per group (32 x 64), stride 2
    (2, 16, 9, 9, 32, 16, 3, 1, False, None, None),            # groups = Cin, two outputs per input channel
    (1, 128, 6, 6, 128, 2, 3, 1, True, None, (136, 3)),        # 64 x 64 groups, odd output offset: direct
]


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("case", GCONV_CASES)
def test_grouped_conv2d(case, dtype):
    """groups not in {1, C} (conv_bn's Conv2d::new_grouped, blocks/conv.rs:51-69)
    against the oracle's grouped conv."""
    import torch
    n, cin, h, w, cout, G, k, s, with_res, xv, yv = case
    rnd = rounder(dtype)
    rng = np.random.default_rng(zlib.crc32(repr(case).encode()))
    x = rnd(rng.standard_normal((n, cin, h, w)).astype(np.float32))
    cg = cin // G
    wt = rnd((rng.standard_normal((cout, cg, k, k)) * np.sqrt(2.0 / (cg * k * k))).astype(np.float32))
    scale = rng.uniform(0.5, 1.5, cout).astype(np.float32)
    shift = rng.normal(0, 0.2, cout).astype(np.float32)
    ho, wo = (h + 2 * (k // 2) - k) // s + 1, (w + 2 * (k // 2) - k) // s + 1
    res = rnd(rng.standard_normal((n, cout, ho, wo)).astype(np.float32)) if with_res else None
    ref = oracle.affine_act(oracle.conv2d(x, wt, s, k // 2, groups=G), scale, shift, 1)
    if with_res:
        ref = ref + res
    xp, xo = xv or (cin, 0)
    yp, yo = yv or (cout, 0)
    xt = to_nhwc(x, dtype, xp, xo)
    yt = torch.full((n, ho, wo, yp), 7.0, dtype=tdtype(dtype), device="cuda")
    rt = to_nhwc(res, dtype, yp, yo) if with_res else None
    ctx().conv2d(vrs.nhwc(xt, cin, xo), dev(vrs.pack_conv_weight(wt, G, None, dtype)), dev(scale), dev(shift),
                 vrs.nhwc(yt, cout, yo), k, s, G, vrs.ACT_SILU, vrs.nhwc(rt, cout, yo) if with_res else None, dtype)
    torch.cuda.synchronize()
    err = rel_err(from_nhwc(yt, cout, yo), ref, FLOOR[dtype])
    assert err < TOL[dtype], err
    if yp > cout:
        rest = torch.cat([yt[..., :yo], yt[..., yo + cout:]], -1).float()
        assert torch.all(rest == 7.0)


def test_grouped_fixture_f32():
    """The reference's g4 grouped-conv fixture (tests/test_conv_grouped_cuda.rs,
    groups 4, 2 input channels per group; 1e-5 absolute) through vrs_conv2d
    with unit scale, zero shift and no activation."""
    import torch
    from golden_io import load
    x = load("conv_grouped/g4/x.bin", (2, 8, 4, 4))
    w = load("conv_grouped/g4/conv_w.bin", (8, 2, 3, 3))
    exp = load("conv_grouped/g4/expected_output.bin", (2, 8, 4, 4))
    xt = to_nhwc(x, vrs.F32)
    yt = torch.zeros((2, 4, 4, 8), dtype=torch.float32, device="cuda")
    one, zero = np.ones(8, np.float32), np.zeros(8, np.float32)
    ctx().conv2d(vrs.nhwc(xt), dev(vrs.pack_conv_weight(w, 4, None, vrs.F32)), dev(one), dev(zero), vrs.nhwc(yt),
                 3, 1, 4, vrs.ACT_NONE, None, vrs.F32)
    torch.cuda.synchronize()
    assert np.max(np.abs(from_nhwc(yt, 8, 0) - exp)) < 1e-5


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("hw", [(20, 20), (7, 5), (4, 4), (26, 26), (30, 22), (40, 40), (1, 9), (13, 1),
                                (20, 20, 64), (9, 11, 96)])
def test_sppf_pool_exact(dtype, hw):
    """bf16 maps up to 1365 pixels run the wave-per-group kernel (four waves
    per workgroup up to 426 pixels when the channel groups come in fours, two
    up to 682, else one; 5 channel groups x 3 images leaves an idle wave), larger ones the plane kernel (float32 40x40 needs its
    160 KB budget); max is exact, so bit-exact
    against the oracle's cascade (with exact ties and signed zeros)."""
    import torch
    h, w = hw[:2]
    rnd = rounder(dtype)
    rng = np.random.default_rng(8)
    n, c = 3, (hw[2] if len(hw) > 2 else 40)
    y = rnd(rng.standard_normal((n, c, h, w)).astype(np.float32))
    y[0, 0] = np.float32(-0.0)
    y[0, 1, :, : max(1, w // 2)] = 1.5   # exact ties
    p1 = oracle.maxpool2d(y); p2 = oracle.maxpool2d(p1); p3 = oracle.maxpool2d(p2)
    buf = torch.zeros((n, h, w, 4 * c + 8), dtype=tdtype(dtype), device="cuda")
    buf[..., 8:8 + c] = to_nhwc(y, dtype)
    ctx().sppf_pool(vrs.nhwc(buf, 4 * c, 8), dtype)
    torch.cuda.synchronize()
    got = from_nhwc(buf, 4 * c, 8)
    assert np.array_equal(got, np.concatenate([y, p1, p2, p3], 1))


@pytest.mark.parametrize("dtype", DT)
def test_upsample_exact(dtype):
    import torch
    rng = np.random.default_rng(9)
    x = rounder(dtype)(rng.standard_normal((2, 16, 5, 3)).astype(np.float32))
    xt = to_nhwc(x, dtype)
    yt = torch.zeros((2, 10, 6, 48), dtype=tdtype(dtype), device="cuda")
    ctx().upsample2x(vrs.nhwc(xt), vrs.nhwc(yt, 16, 24), dtype)
    torch.cuda.synchronize()
    assert np.array_equal(from_nhwc(yt, 16, 24), oracle.upsample_nearest(x))
    assert torch.all(yt[..., :24] == 0) and torch.all(yt[..., 40:] == 0)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("shape", [
    (2, 2, 4, 4), (2, 4, 20, 20), (1, 1, 7, 9),
    # bf16 kernel choice: LDS-resident heads (N <= 512) in tiles of 7 query
    # tiles (few heads: 1, 2 or 3 workgroups per head), one workgroup per head
    # of 13 or 16 query tiles (once the 7-tile workgroups would take more than
    # one round over the CUs: 160 and 256 heads), and the streamed kernel
    # beyond 512 keys
    (3, 2, 13, 17), (2, 4, 23, 22), (40, 4, 20, 20), (64, 4, 20, 20), (64, 4, 22, 22), (1, 1, 24, 24)])
def test_psa_attention(dtype, shape):
    import torch
    b, heads, h, w = shape
    rnd = rounder(dtype)
    rng = np.random.default_rng(10)
    qkv = rnd(rng.standard_normal((b, heads * 128, h, w)).astype(np.float32))
    c = heads * 64
    pe_w = rnd((rng.standard_normal((c, 1, 3, 3)) * 0.3).astype(np.float32))
    pe_s = rng.uniform(0.5, 1.5, c).astype(np.float32)
    pe_t = rng.normal(0, 0.1, c).astype(np.float32)
    att = oracle.psa_attention(qkv, heads, 32, 64)
    v = np.ascontiguousarray(qkv.reshape(b, heads, 128, h, w)[:, :, 64:].reshape(b, c, h, w))
    ref = att + oracle.affine_act(oracle.conv2d(v, pe_w, 1, 1, groups=c), pe_s, pe_t, 0)
    qt = to_nhwc(qkv, dtype)
    ot = torch.zeros((b, h, w, c), dtype=tdtype(dtype), device="cuda")
    ctx().psa_attention(vrs.nhwc(qt), dev(vrs.pack_conv_weight(pe_w, c, 1, dtype)), dev(pe_s), dev(pe_t),
                        vrs.nhwc(ot), heads, dtype)
    torch.cuda.synchronize()
    err = rel_err(from_nhwc(ot), ref, FLOOR[dtype])
    assert err < TOL[dtype], err


def test_detect_decode_grid_fixture():
    import torch
    from golden_io import load
    B, A = 2, 16
    boxes = dev(load("detect_decode/raw_boxes.bin", (B, 4, A)))
    out = torch.empty_like(boxes)
    ctx().detect_decode_grid(boxes, dev(load("detect_decode/anchor_x.bin")), dev(load("detect_decode/anchor_y.bin")),
                             dev(load("detect_decode/strides.bin")), out)
    torch.cuda.synchronize()
    assert np.max(np.abs(out.cpu().numpy() - load("detect_decode/expected.bin", (B, 4, A)))) < 1e-4


def _check_post(got, ref, thr_tol=1e-6):
    count, sc, cl, an, xy = [g.cpu().numpy() for g in got]
    rc, rs, rcl, ran, rxy = ref
    assert np.array_equal(count, rc)
    for b in range(len(count)):
        k = count[b]
        assert np.allclose(sc[b, :k], rs[b, :k], rtol=thr_tol, atol=0)
        # identical order / class wherever neighbouring scores differ by more than the tolerance
        same = np.abs(np.diff(rs[b, :k])) > 1e-6 * np.abs(rs[b, 1:k])
        ok = np.ones(k, bool)
        ok[1:] &= same
        ok[:-1] &= same
        assert np.array_equal(an[b, :k][ok], ran[b, :k][ok])
        assert np.array_equal(cl[b, :k][ok], rcl[b, :k][ok])
        assert np.allclose(xy[b, :k][ok], rxy[b, :k][ok], rtol=1e-6, atol=1e-4)
        assert np.all(an[b, k:] == -1)


@pytest.mark.parametrize("img,nc,thr,max_det", [(64, 5, 0.25, 50), (640, 80, 0.25, 300), (640, 80, 0.001, 1024),
                                                (96, 3, 0.999, 7)])
def test_detect_postprocess(img, nc, thr, max_det):
    rng = np.random.default_rng(11)
    strides = (8, 16, 32)
    A = sum((img // s) ** 2 for s in strides)
    B = 3
    boxes = rng.uniform(0, 5, (B, 4 * A)).astype(np.float32)
    scores = rng.normal(-2, 2, (B, nc * A)).astype(np.float32)
    scores[0, : nc * 10] = 4.0  # exact ties in classes and across anchors
    got = ctx().detect_postprocess(dev(boxes), dev(scores), nc, img, img, strides, thr, max_det)
    import torch
    torch.cuda.synchronize()
    ref = oracle.detect_postprocess(boxes, scores, nc, img, img, strides, thr, max_det)
    _check_post(got, ref)


def test_detect_postprocess_empty():
    rng = np.random.default_rng(12)
    A = 21
    boxes = rng.uniform(0, 5, (2, 4 * A)).astype(np.float32)
    scores = np.full((2, 3 * A), -30.0, np.float32)
    count, sc, cl, an, xy = ctx().detect_postprocess(dev(boxes), dev(scores), 3, 32, 32, (8, 16, 32), 0.25, 10)
    assert count.cpu().numpy().tolist() == [0, 0]
    assert np.all(an.cpu().numpy() == -1)


def test_detect_unletterbox():
    """Letterbox pixels -> boxes normalised to the original image, bit-exact
    against the oracle's float32 restatement; slots past count are zero.  The
    original sizes cover landscape, portrait, square, sizes whose scaled side
    rounds, and an image smaller than the letterbox."""
    import torch
    rng = np.random.default_rng(5)
    wh = np.array([[1920, 1080], [480, 640], [640, 640], [333, 777], [1001, 999], [37, 100]], np.int32)
    B, max_det = len(wh), 300
    xywh = rng.uniform(0, 640, (B, max_det, 4)).astype(np.float32)
    count = np.array([300, 17, 0, 1, 250, 300], np.int32)
    got = ctx().detect_unletterbox(dev(count), dev(xywh), dev(wh), 640)
    torch.cuda.synchronize()
    ref = oracle.detect_unletterbox(count, xywh, wh, 640)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    with pytest.raises(vrs.VrsError):
        ctx().detect_unletterbox(dev(count), dev(xywh), dev(wh), 0)


LB_SIZES = [(1280, 720), (640, 640), (517, 333), (333, 517), (1000, 37), (5, 3), (1, 1), (17, 2000), (4000, 100),
            (1920, 1080), (639, 641), (2, 1), (100, 100), (64, 48), (3000, 3000), (701, 299), (8, 8), (1279, 719),
            (333, 333), (50, 2000), (2560, 1440), (2600, 100), (5120, 300), (6000, 200)]


def test_letterbox():
    """Letterbox preprocessing of 24 images of mixed sizes, bit-exact against
    the oracle's two-pass restatement of the Triangle resize, through every
    kernel: enlargements and shrinks up to 2x (staged, 64-wide tiles), up to 4x
    (1920 and exactly 4x at 2560 wide), up to 8x (2600, 4000, exactly 8x at
    5120 wide: 32-wide tiles) and beyond (6000 wide: direct kernel); the
    identity, 1x1, thin strips, saturated regions, odd byte offsets."""
    import torch
    rng = np.random.default_rng(9)
    imgs = []
    for i, (w, h) in enumerate(LB_SIZES):
        im = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
        if i % 4 == 1:   # saturated blocks exercise the clamp
            im[: h // 2, : w // 2] = 255
            im[h // 2:, w // 2:] = 0
        imgs.append(im)
    offs, parts, pos = [], [], 0
    for im in imgs:
        parts.append(np.zeros(1 + pos % 3, np.uint8))   # odd starting offsets
        pos += parts[-1].size
        offs.append(pos)
        parts.append(im.reshape(-1))
        pos += im.size
    flat = dev(np.concatenate(parts))
    got = ctx().letterbox(flat, offs, LB_SIZES, 640)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    for i, im in enumerate(imgs):
        ref = oracle.letterbox(im, 640)
        assert np.array_equal(got[i].view(np.uint32), ref.view(np.uint32)), (i, LB_SIZES[i])


def test_letterbox_rejections():
    """Host-side checks, no launch: empty images, images past the buffer, and
    shrinks beyond 62x per axis (bounded filter windows)."""
    import torch
    flat = torch.zeros(4000 * 100 * 3, dtype=torch.uint8, device="cuda")
    out = torch.empty(1, 3, 64, 64, device="cuda")
    for offs, wh, S in [([0], [(0, 10)], 64), ([1], [(4000, 100)], 640), ([-1], [(10, 10)], 64),
                        ([0], [(4000, 100)], 64)]:
        with pytest.raises(vrs.VrsError):
            ctx().letterbox(flat, offs, wh, S, out=out)
    ctx().letterbox(flat, [0], [(4000, 100)], 65, out=torch.empty(1, 3, 65, 65, device="cuda"))   # 61.5x: accepted
    torch.cuda.synchronize()


@pytest.mark.parametrize("cfg", [
    (2, 30, 4, [(16, 16), (8, 8), (4, 4), (2, 2)], 4),   # level-split kernel (one wave per level)
    (1, 6, 16, [(9, 9), (5, 5), (3, 3), (2, 2)], 4),     # unrolled 4x4 kernel (> 8 heads)
    (1, 7, 8, [(13, 11), (7, 6)], 3),                    # generic kernel
    (1, 5, 8, [(80, 80), (40, 40), (20, 20), (10, 10)], 4),  # BASELINE config 4 level shapes
])
def test_msda(cfg):
    import torch
    from test_oracle_golden import msda_inputs
    B, Q, heads, shapes, P = cfg
    value, ref, off, attw = msda_inputs(B, Q, heads, 32, shapes, P)
    exp = oracle.msda(value, shapes, ref, off, attw)
    out = torch.empty((B, Q, heads * 32), dtype=torch.float32, device="cuda")
    ctx().msda(dev(value), shapes, dev(ref), dev(off), dev(attw), out)
    torch.cuda.synchronize()
    assert rel_err(out.cpu().numpy(), exp, FLOOR[vrs.F32]) < 1e-4


def test_errors_are_reported_not_fatal():
    import torch
    C = ctx()
    x = torch.zeros((1, 4, 4, 12), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((1, 4, 4, 16), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(16 * 12, dtype=torch.bfloat16, device="cuda")
    s = torch.ones(16, device="cuda")
    with pytest.raises(vrs.VrsError) as e:  # Cin 12 is not a multiple of 8
        C.conv2d(vrs.nhwc(x), w, s, s, vrs.nhwc(y), 1, 1, 1, vrs.ACT_SILU, None, vrs.BF16)
    assert e.value.code == -2
    with pytest.raises(vrs.VrsError) as e:  # groups must divide both channel counts
        C.conv2d(vrs.nhwc(y), w, s, s, vrs.nhwc(y), 3, 1, 3, vrs.ACT_SILU, None, vrs.BF16)
    assert e.value.code == -2
