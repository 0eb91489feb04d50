"""GPU parity of vrs_conv_stem_pair (model.0 + model.1 of YOLO26 m/l in one
kernel) against the CPU oracle and against the two-kernel path.

The oracle check is the north_star's bfloat16 bar (2e-2 relative, floor 0.1
rms, as the single-op tests): the stem output is rounded to bfloat16 before
model.1, as the unfused network stores it.  The two-kernel comparison
(vrs_conv_stem, then vrs_conv2d on the 128x128 tile with 64-deep K steps) is
bit-exact: the pair kernel runs the same MFMA instructions in the same K order
and the same epilogue arithmetic.

Shapes cover the walker's edges: an output narrower than one 32-column strip,
a last strip with 1 valid column and a last row pair with 1 valid row, a
grid with several steps (and strip changes) per workgroup, and the bench
configuration's 64 x 640 x 640 (checked against the two-kernel path only)."""
import numpy as np
import pytest

import oracle
from gpu_util import bf16_round, ctx, dev, from_nhwc, rel_err, vrs

pytestmark = pytest.mark.gpu


def _params(rng):
    w0 = bf16_round((rng.standard_normal((64, 3, 3, 3)) * np.sqrt(2.0 / 27)).astype(np.float32))
    s0 = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    t0 = rng.normal(0, 0.2, 64).astype(np.float32)
    w1 = bf16_round((rng.standard_normal((128, 64, 3, 3)) * np.sqrt(2.0 / 576)).astype(np.float32))
    s1 = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    t1 = rng.normal(0, 0.2, 128).astype(np.float32)
    return w0, s0, t0, w1, s1, t1


def _run(x, prm, y_pitch=128, y_off=0):
    """Pair kernel and two-kernel path on the same inputs; returns both
    NHWC outputs (the pair's in a view of pitch y_pitch at channel y_off)."""
    import torch
    w0, s0, t0, w1, s1, t1 = prm
    n, _, h, w = x.shape
    C = ctx()
    xd = dev(x)
    w0p, w1p = dev(vrs.pack_stem_weight(w0, vrs.BF16)), dev(vrs.pack_conv_weight(w1, 1, 64, vrs.BF16))
    s0d, t0d, s1d, t1d = dev(s0), dev(t0), dev(s1), dev(t1)
    h0, w0o = (h - 1) // 2 + 1, (w - 1) // 2 + 1
    h1, w1o = (h0 - 1) // 2 + 1, (w0o - 1) // 2 + 1
    yp = torch.full((n, h1, w1o, y_pitch), 7.0, dtype=torch.bfloat16, device="cuda")
    C.conv_stem_pair(xd, w0p, s0d, t0d, w1p, s1d, t1d, vrs.nhwc(yp, 128, y_off))
    st = torch.empty((n, h0, w0o, 64), dtype=torch.bfloat16, device="cuda")
    yr = torch.empty((n, h1, w1o, 128), dtype=torch.bfloat16, device="cuda")
    C.conv_stem(xd, w0p, s0d, t0d, vrs.nhwc(st), vrs.ACT_SILU, vrs.BF16)
    C.conv2d(vrs.nhwc(st), w1p, s1d, t1d, vrs.nhwc(yr), 3, 2, 1, vrs.ACT_SILU, None, vrs.BF16,
             tile=vrs.TILE_128x128)
    torch.cuda.synchronize()
    return yp, yr


def _oracle(x, prm):
    w0, s0, t0, w1, s1, t1 = prm
    s = bf16_round(oracle.affine_act(oracle.conv2d(x, w0, 2, 1), s0, t0, 1))
    return oracle.affine_act(oracle.conv2d(s, w1, 2, 1), s1, t1, 1)


@pytest.mark.parametrize("shape", [
    (2, 64, 64),      # output 16 x 16: one strip, half of it past the edge
    (6, 250, 252),    # output 63 x 63: last strip 31 columns, last row pair 1 row
    (8, 320, 320),    # 960 steps on 256 workgroups: 3-4 steps each, strip changes mid-run
    (3, 36, 8),       # output 9 x 2
])
def test_stem_pair_matches_oracle_and_two_kernels(shape):
    import torch
    n, h, w = shape
    rng = np.random.default_rng(h * 1000 + w)
    x = bf16_round(rng.uniform(0, 1, (n, 3, h, w)).astype(np.float32))
    prm = _params(rng)
    yp, yr = _run(x, prm, y_pitch=144, y_off=8)
    got = yp[..., 8:136]
    assert torch.equal(got, yr), int((got != yr).sum())
    rest = torch.cat([yp[..., :8], yp[..., 136:]], -1).float()
    assert torch.all(rest == 7.0)
    err = rel_err(from_nhwc(yp, 128, 8), _oracle(x, prm), 1e-1)
    assert err < 2e-2, err


def test_stem_pair_bench_size_matches_two_kernels():
    """64 x 640 x 640 (the bench configuration): 100 steps per workgroup."""
    import torch
    rng = np.random.default_rng(5)
    x = rng.uniform(0, 1, (64, 3, 640, 640)).astype(np.float32)
    yp, yr = _run(x, _params(rng))
    assert torch.equal(yp, yr), int((yp != yr).sum())


def test_stem_pair_rejections():
    import torch
    rng = np.random.default_rng(1)
    w0, s0, t0, w1, s1, t1 = (dev(a) for a in _params(rng))
    C = ctx()
    x = dev(np.zeros((1, 3, 16, 18), np.float32))   # width not a multiple of 4
    y = torch.zeros((1, 4, 5, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(vrs.VrsError) as e:
        C.conv_stem_pair(x, w0, s0, t0, w1, s1, t1, vrs.nhwc(y))
    assert e.value.code == -3
    x = dev(np.zeros((1, 3, 16, 16), np.float32))
    y = torch.zeros((1, 4, 4, 128), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(vrs.VrsError) as e:   # no float32 build
        C.conv_stem_pair(x, w0, s0, t0, w1, s1, t1, vrs.nhwc(y), dtype=vrs.F32)
    assert e.value.code == -3
    with pytest.raises(vrs.VrsError) as e:   # SiLU layers only
        C.conv_stem_pair(x, w0, s0, t0, w1, s1, t1, vrs.nhwc(y), act=vrs.ACT_NONE)
    assert e.value.code == -3
    y = torch.zeros((1, 4, 4, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(vrs.VrsError) as e:   # 128 output channels
        C.conv_stem_pair(x, w0, s0, t0, w1, s1, t1, vrs.nhwc(y))
    assert e.value.code == -2
