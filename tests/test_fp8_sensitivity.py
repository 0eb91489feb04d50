"""Why the fp8 network cannot be held to the bf16 end-to-end bar (CPU only).

Every fp8 conv of the device is held, layer by layer, to the single-kernel
bar against the oracle conv on the same dequantised e4m3 operands
(tests/test_gpu_layers.py).  End to end the device differs from the
precision-matched emulation by about as much as the emulation differs from
float32.  The cause is e4m3 rounding itself: an activation that is one bf16
ulp away on the two sides (the device and the oracle sum in different orders)
sometimes rounds to the neighbouring e4m3 value, a step of 2^-3 relative, and
those steps compound over the ~90 quantised layers.  This test shows it with
the oracle alone: perturbing 0.1 % of the bf16 activations of the emulation
by one ulp moves its outputs by several percent, while the same perturbation
moves the bf16 emulation by well under one percent.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "vision-rs_amd"))

from oracle import yolo26 as Y  # noqa: E402
from gpu_util import bf16_round  # noqa: E402
from golden_io import seeded_params  # noqa: E402
import vrs  # noqa: E402


def fp8_eligible(specs):
    """The convs a VRS_FP8 model runs on e4m3: dense, Cin % 64 == 0, not the
    stem and not a fused-upsample 1x1 (model.13.cv1, model.16.cv1)."""
    out = set()
    for name, shape in specs:
        if len(shape) != 4 or ".bn." in name:
            continue
        pre = name[: -len(".conv.weight")] if name.endswith(".conv.weight") else name[: -len(".weight")]
        cout, cin_g = shape[0], shape[1]
        if cin_g == 1 and cout > 1:          # depthwise
            continue
        if pre in ("model.0", "model.13.cv1", "model.16.cv1") or cin_g % 64:
            continue
        out.add(pre)
    return out


def normwise(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def one_ulp_flips(frac, seed):
    """act_q that rounds to bf16 and then moves a random `frac` of the
    elements one bf16 ulp up or down."""
    rng = np.random.default_rng(seed)

    def q(t):
        u = bf16_round(t).view(np.uint32).astype(np.int64)
        pick = rng.random(u.shape) < frac
        step = np.where(rng.random(u.shape) < 0.5, 0x10000, -0x10000)
        return np.where(pick, u + step, u).astype(np.uint32).view(np.float32)
    return q


def test_e4m3_emulation_amplifies_one_ulp_differences():
    S = 160
    desc = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="m", one2one=True)
    specs = vrs.Model(None, desc, 1, S, S, vrs.BF16, 1e-3).params()
    P32 = seeded_params(specs, 0, bn="identity")
    P = {k: (bf16_round(v) if v.ndim == 4 else v) for k, v in P32.items()}
    x = bf16_round(np.random.default_rng(7).uniform(0, 1, (1, 3, S, S)).astype(np.float32))
    net = Y.yolo26(80, "m")
    elig = fp8_eligible(specs)
    assert len(elig) == 90
    steps = Y.fp8_steps(net, Y.Params(P, eps=1e-3, act_q=bf16_round), x, elig)
    assert set(steps) == elig
    ref = net(Y.Params(P32, eps=1e-3), x)
    e8 = net(Y.Params(P, eps=1e-3, act_q=bf16_round, fp8=steps), x)
    e8p = net(Y.Params(P, eps=1e-3, act_q=one_ulp_flips(1e-3, 11), fp8=steps), x)
    e16 = net(Y.Params(P, eps=1e-3, act_q=bf16_round), x)
    e16p = net(Y.Params(P, eps=1e-3, act_q=one_ulp_flips(1e-3, 11)), x)
    for i, name in enumerate(("boxes", "scores")):
        d8, d16 = normwise(e8p[i], e8[i]), normwise(e16p[i], e16[i])
        q8, q16 = normwise(e8[i], ref[i]), normwise(e16[i], ref[i])
        print(f"{name}: fp8 emulation vs float32 {q8:.3e}, one-ulp flips move it by {d8:.3e}; "
              f"bf16 emulation vs float32 {q16:.3e}, moved by {d16:.3e}")
        # e4m3 rounding turns 0.1 % one-ulp flips into a several-percent change
        # of the outputs, the same order as its own error against float32 ...
        assert d8 > 3e-2 and d8 > 0.3 * q8
        # ... while bf16 storage absorbs them
        assert d16 < 1e-2 and d16 < 0.2 * d8
