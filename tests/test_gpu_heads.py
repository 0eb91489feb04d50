"""GPU parity of the Detect head as its own block, of the YOLO26 variants
the other tests do not run numerically (s, l, x, and the OneToMany head), and
of the detection contract on logits planted to have wide margins.

* VRS_BLOCK_DETECT: detect::<D>(nc, &ch, head) (blocks/detect.rs:108-172) on
  three feature maps, both heads (DetectHead::OneToOne -> one2one_cv2/3,
  OneToMany -> cv2/3), float32 at 1e-4 and bfloat16 at the multi-layer bf16
  bar, against oracle/yolo26.py's detect.
* YOLO26 s / l / x (yolo26/mod.rs:70-100: x is width 1.5, l and x depth 1.0,
  so every C3k2 has two blocks) and n with the OneToMany head, float32
  against the oracle: normwise relative error < 1e-4 (the north_star's fp32
  tolerance), and elementwise (floor 0.1 * rms) < 1e-3.  The elementwise
  figure is the YOLO26n config-1 test's 1e-4 bar loosened tenfold: two
  float32 implementations that sum K = 9 * Cin products per output in
  different orders drift apart by ~1e-7 relative per layer, and the wider
  (x: up to 9 * 768 per output) and deeper (l, x: two blocks per C3k2)
  networks with random BN statistics carry that drift through ~150 layers
  (measured: YOLO26s at 128x128 2e-4 / 6e-4 elementwise).
* Planted margins: with seeded Kaiming weights and identity BN the class
  logits of YOLO26m spread by only ~1e-2, so the argmax/top-k contract
  ("identical wherever the margin exceeds the tolerance") has few anchors to
  check.  Scaling the class output convs (conv_plain, blocks/conv.rs:90-99)
  so the logits spread by ~3, with a bias of -10 so that a few dozen anchors
  per image clear the 0.25 threshold at distinct scores, gives thousands of
  anchors and several ranks to hold to it.
"""
import numpy as np
import pytest

import oracle
from oracle import yolo26 as Y
from gpu_util import bf16_round, ctx, dev, rel_err, vrs
from golden_io import seeded_params
from test_gpu_layers import detection_checks, normwise

pytestmark = pytest.mark.gpu


def _forward(m, x):
    import torch
    outs = m.forward(dev(x))
    torch.cuda.synchronize()
    return [o.cpu().numpy() for o in outs]


def bf16_block_errors(got, ref):
    """(normwise relative error, max elementwise error over max(|ref|, rms))."""
    return normwise(got, ref), rel_err(got, ref, 1.0)


@pytest.mark.parametrize("dtype,one2one", [(vrs.F32, True), (vrs.F32, False), (vrs.BF16, True)],
                         ids=["f32-one2one", "f32-one2many", "bf16-one2one"])
def test_detect_block_vs_oracle(dtype, one2one):
    chs, nc, B, h = (64, 128, 256), 80, 2, 32
    desc = vrs.block(vrs.BLOCK_DETECT, chs[0], nc=nc, one2one=one2one, ch=chs)
    m = vrs.Model(ctx(), desc, B, h, h, dtype, 1e-3)
    names = [n for n, _ in m.params()]
    head = "one2one_cv" if one2one else "cv"
    assert all(n.startswith((f"{head}2.", f"{head}3.")) for n in names), names[:4]
    P = seeded_params(m.params(), 5, bn="random")
    rng = np.random.default_rng(6)
    feats = [rng.standard_normal((B, c, h >> i, h >> i)).astype(np.float32) for i, c in enumerate(chs)]
    if dtype == vrs.BF16:
        P = {k: (bf16_round(v) if v.ndim == 4 else v) for k, v in P.items()}
        feats = [bf16_round(f) for f in feats]
    m.load(P)
    A = h * h + (h // 2) ** 2 + (h // 4) ** 2
    assert m.output_shapes() == [(B, 4 * A), (B, nc * A)]
    x = np.concatenate([f.reshape(-1) for f in feats])
    boxes, scores = _forward(m, x)
    act_q = bf16_round if dtype == vrs.BF16 else None
    rb, rs = Y.detect(nc, list(chs), one2one)(Y.Params(P, eps=1e-3, act_q=act_q), "", feats)
    for got, ref, name in ((boxes, rb, "boxes"), (scores, rs, "scores")):
        if dtype == vrs.F32:
            err = rel_err(got, ref, 1e-1)
            print(f"detect block f32 {name}: max rel err {err:.2e}")
            assert err < 1e-4, (name, err)
        else:
            nw, el = bf16_block_errors(got, ref)
            print(f"detect block bf16 {name}: normwise {nw:.2e}, elementwise {el:.2e}")
            assert nw < 2e-2 and el < 5e-2, (name, nw, el)


@pytest.mark.parametrize("variant,one2one,size", [("s", True, 128), ("l", True, 128), ("x", True, 128),
                                                  ("n", False, 160)],
                         ids=["s", "l", "x", "n-one2many"])
def test_yolo26_variant_f32_vs_oracle(variant, one2one, size):
    desc = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant=variant, one2one=one2one)
    m = vrs.Model(ctx(), desc, 1, size, size, vrs.F32, 1e-3)
    P = seeded_params(m.params(), 0, bn="random")
    m.load(P)
    x = np.random.default_rng(2).uniform(0, 1, (1, 3, size, size)).astype(np.float32)
    boxes, scores = _forward(m, x)
    rb, rs = Y.yolo26(80, variant, one2one)(Y.Params(P, eps=1e-3), x)
    A = sum((size // s) ** 2 for s in (8, 16, 32))
    assert boxes.shape == (1, 4 * A) and scores.shape == (1, 80 * A)
    eb, es = rel_err(boxes, rb, 1e-1), rel_err(scores, rs, 1e-1)
    nb, ns = normwise(boxes, rb), normwise(scores, rs)
    print(f"yolo26{variant} {'one2one' if one2one else 'one2many'} f32 {size}: normwise boxes {nb:.2e} "
          f"scores {ns:.2e}; elementwise boxes {eb:.2e} scores {es:.2e}")
    assert nb < 1e-4 and ns < 1e-4
    assert eb < 1e-3 and es < 1e-3


# class-output conv weight factors that spread each scale's logits by ~3 at
# seed 0 (their spread is 0.0131, 0.0026 and 0.0121 at 320x320 unscaled)
PLANT_SCALE = (3.0 / 0.0131, 3.0 / 0.00256, 3.0 / 0.0121)
PLANT_BIAS = -10.0


def test_yolo26m_bf16_planted_margins():
    x32 = np.random.default_rng(7).uniform(0, 1, (2, 3, 320, 320)).astype(np.float32)
    x = bf16_round(x32)
    desc = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="m", one2one=True)
    m = vrs.Model(ctx(), desc, 2, 320, 320, vrs.BF16, 1e-3)
    P32 = seeded_params(m.params(), 0, bn="identity")
    for i, k in enumerate(PLANT_SCALE):
        P32[f"model.23.one2one_cv3.{i}.2.weight"] = P32[f"model.23.one2one_cv3.{i}.2.weight"] * np.float32(k)
        P32[f"model.23.one2one_cv3.{i}.2.bias"] = np.full(80, PLANT_BIAS, np.float32)
    P = {k: (bf16_round(v) if v.ndim == 4 else v) for k, v in P32.items()}
    m.load(P)
    boxes, scores = _forward(m, x)
    rb, rs = Y.yolo26(80, "m")(Y.Params(P32, eps=1e-3), x32)
    eb, es = normwise(boxes, rb), normwise(scores - PLANT_BIAS, rs - PLANT_BIAS)
    n_am, mism, n_tk, topk_bad, counts = detection_checks(boxes, scores, rb, rs, 320)
    print(f"planted: normwise boxes {eb:.2e} logits {es:.2e}; argmax mismatches {mism} of {n_am} checked anchors; "
          f"top-k mismatches {topk_bad} of {n_tk} separated ranks; detections {counts[0]} vs {counts[1]}")
    assert eb < 2e-2 and es < 2e-2
    assert n_am > 3000 and mism == 0          # of 2 x 2100 anchors
    assert n_tk >= 2 and topk_bad == 0
    assert min(counts[0]) >= 20
