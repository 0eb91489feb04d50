"""Pin the CPU oracle against the reference's own golden vectors (tests/golden/,
copied from the reference's tests/fixtures) and, where no fixture exists,
against independent library routines / closed forms.

Tolerances follow the reference tests that consume each fixture:
  conv_grouped 1e-5 abs (tests/test_conv_grouped_cuda.rs:47)
  conv_yolo26 1e-4 abs (tests/test_conv_yolo26.rs:250)
  c3k2 / c2psa / sppf / detect 1e-3 abs (tests/test_c3k2_variants_cuda.rs:47, ...)
  detect_decode 1e-4 abs (tests/test_detect_decode.rs:91)
All of those fixtures were made with PyTorch's BN eps 1e-5 (e.g. tests/test_c2psa_cuda.rs:103).
"""
import numpy as np
import pytest

import oracle
from oracle import yolo26 as Y
from golden_io import block_params, load

EPS_FIXTURE = 1e-5


def _shapes(family, table):
    """table: prefix -> k; Cin/g is derived from the file size."""
    import os
    from golden_io import GOLDEN, fixture_prefix_to_name
    shapes = {}
    for f in os.listdir(os.path.join(GOLDEN, family)):
        if not f.endswith("_conv_w.bin"):
            continue
        pre = f[: -len("_conv_w.bin")]
        name = fixture_prefix_to_name(pre)
        k = table.get(name, 1)
        w = load(f"{family}/{f}")
        co = load(f"{family}/{pre}_bn_w.bin").shape[0]
        shapes[name] = (co, w.size // (co * k * k), k, k)
    return shapes


# ---------------------------------------------------------------- conv / bn --

@pytest.mark.parametrize("sub,cin,cout,g", [("depthwise", 128, 128, 128), ("g4", 8, 8, 4)])
def test_conv_grouped(sub, cin, cout, g):
    """The reference's grouped-conv fixtures against the oracle (the GPU runs
    the same fixtures: test_gpu_blocks.test_depthwise_fixture_f32 and
    test_gpu_ops.test_grouped_fixture_f32)."""
    x = load(f"conv_grouped/{sub}/x.bin", (2, cin, 4, 4))
    w = load(f"conv_grouped/{sub}/conv_w.bin", (cout, cin // g, 3, 3))
    exp = load(f"conv_grouped/{sub}/expected_output.bin", (2, cout, 4, 4))
    y = oracle.conv2d(x, w, stride=1, pad=1, groups=g)
    assert np.max(np.abs(y - exp)) < 1e-5


def test_grouped_weight_pack_layout():
    """groups not in {1, C}: the packer writes each output channel's Cin/groups
    inputs in the dense order [Cout][k][k][Cin/groups] (the OIHW weight with
    I moved last); channel padding and Cout not divisible by groups are refused.
    Depthwise (groups == Cout, one input per group) stays tap-major."""
    from gpu_util import vrs
    w = load("conv_grouped/g4/conv_w.bin", (8, 2, 3, 3))
    got = np.frombuffer(vrs.pack_conv_weight(w, groups=4, dtype=vrs.F32).tobytes(), np.float32)
    assert np.array_equal(got, w.transpose(0, 2, 3, 1).ravel())
    got = np.frombuffer(vrs.pack_conv_weight(w, groups=4).tobytes(), np.uint16)
    assert np.array_equal(got, (bf16_bits(w.transpose(0, 2, 3, 1).ravel())))
    for kw in ({"groups": 4, "cin_pad": 8}, {"groups": 3}):
        with pytest.raises(vrs.VrsError) as e:
            vrs.pack_conv_weight(w, **kw)
        assert e.value.code == -1   # VRS_EINVAL
    wd = load("conv_grouped/depthwise/conv_w.bin", (128, 1, 3, 3))
    got = np.frombuffer(vrs.pack_conv_weight(wd, groups=128, dtype=vrs.F32).tobytes(), np.float32)
    assert np.array_equal(got, wd.reshape(128, 9).T.ravel())


def bf16_bits(v):
    """float32 -> bfloat16 bits, round to nearest even (finite inputs)."""
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def test_conv_stem_train_bn():
    x = load("conv_yolo26/x.bin", (2, 3, 16, 16))
    w = load("conv_yolo26/conv_weight.bin", (16, 3, 3, 3))
    y = oracle.conv2d(x, w, stride=2, pad=1)
    oracle.bn_train(y, load("conv_yolo26/bn_weight.bin"), load("conv_yolo26/bn_bias.bin"), EPS_FIXTURE)
    y = oracle.silu(y)
    exp = load("conv_yolo26/expected_output.bin", (2, 16, 8, 8))
    assert np.max(np.abs(y - exp)) < 1e-4


def test_conv_matches_torch_strided():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 24, 13, 11)).astype(np.float32)
    for k, s, g in [(3, 2, 1), (1, 1, 1), (3, 1, 24), (3, 1, 1), (1, 2, 1)]:
        w = rng.standard_normal((16 if g == 1 else 24, 24 // g, k, k)).astype(np.float32)
        b = rng.standard_normal(w.shape[0]).astype(np.float32)
        y = oracle.conv2d(x, w, stride=s, pad=k // 2, groups=g, bias=b)
        t = torch.nn.functional.conv2d(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(b),
                                       stride=s, padding=k // 2, groups=g).numpy()
        assert np.allclose(y, t, rtol=1e-4, atol=1e-4), (k, s, g)


def test_bn_fold_closed_form():
    # identity BN with eps 1e-3 gives scale exactly 1/sqrt(1.001), shift 0
    s, t = oracle.bn_fold(np.ones(4, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32),
                          np.ones(4, np.float32), 1e-3)
    assert np.all(s == np.float32(1.0) / np.sqrt(np.float32(1.001)))
    assert np.all(t == 0)
    # non-trivial: a planted sign error (beta + scale*mean) would fail this
    s, t = oracle.bn_fold(np.array([2.], np.float32), np.array([0.5], np.float32),
                          np.array([3.], np.float32), np.array([3.999], np.float32), 1e-3)
    assert abs(s[0] - 1.0) < 1e-6 and abs(t[0] - (0.5 - 3.0)) < 1e-6


# ------------------------------------------------------------- activations --

@pytest.mark.parametrize("fam,fn", [("silu_4d", "silu"), ("sigmoid_4d", "sigmoid")])
def test_activations(fam, fn):
    x = load(f"{fam}/x.bin")
    exp = load(f"{fam}/expected_forward.bin")
    assert np.max(np.abs(getattr(oracle, fn)(x) - exp)) < 1e-5


def test_concat_upsample():
    x0 = load("concat_upsample/x0.bin", (2, 16, 4, 4))
    x1 = load("concat_upsample/x1.bin", (2, 16, 4, 4))
    assert np.array_equal(np.concatenate([x0, x1], 1), load("concat_upsample/expected_cat.bin", (2, 32, 4, 4)))
    xu = load("concat_upsample/xu.bin", (2, 16, 4, 4))
    assert np.array_equal(oracle.upsample_nearest(xu), load("concat_upsample/expected_up.bin", (2, 16, 8, 8)))


def test_maxpool_matches_torch_edges():
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(2).standard_normal((2, 5, 11, 9)).astype(np.float32)
    y = oracle.maxpool2d(x, 5, 1, 2)
    t = torch.nn.functional.max_pool2d(torch.from_numpy(x), 5, 1, 2).numpy()
    assert np.array_equal(y, t)
    # cascade identity used by the fused SPPF kernel: max5(max5(y)) == max9(y) (clipped windows)
    assert np.array_equal(oracle.maxpool2d(y, 5, 1, 2), oracle.maxpool2d(x, 9, 1, 4))


# ------------------------------------------------------------------ blocks --

C3K2_CASES = [
    # dir, (c_in, c_out, c3k, shortcut, e) -- tests/fixtures/c3k2_yolo26/generate_all.py:211-233
    ("", (32, 64, False, False, 0.25)),
    ("shortcut", (32, 64, False, True, 0.25)),
    ("deep_sf", (128, 128, True, False, 0.5)),
    ("deep_st", (128, 128, True, True, 0.5)),
    ("head_sf", (384, 128, False, False, 0.5)),
    ("head_st", (384, 256, True, True, 0.5)),
]


def c3k2_fixture(sub):
    fam = f"c3k2_yolo26/{sub}".rstrip("/")
    c_in, c_out, c3k, sc, e = dict(C3K2_CASES)[sub]
    ktab = {"m.0.cv1": 3, "m.0.cv2": 3} if not c3k else {
        "m.0.m.0.cv1": 3, "m.0.m.0.cv2": 3, "m.0.m.1.cv1": 3, "m.0.m.1.cv2": 3}
    P = Y.Params(block_params(fam, _shapes(fam, ktab)), eps=EPS_FIXTURE)
    x = load(f"{fam}/x.bin", (2, c_in, 4, 4))
    exp = load(f"{fam}/expected_output.bin", (2, c_out, 4, 4))
    return P, x, exp, (c_in, c_out, c3k, sc, e)


@pytest.mark.parametrize("sub", [c[0] for c in C3K2_CASES])
def test_c3k2_variants(sub):
    P, x, exp, (c_in, c_out, c3k, sc, e) = c3k2_fixture(sub)
    y = Y.c3k2(c_in, c_out, 1, c3k, sc, e)(P, "", x)
    assert np.max(np.abs(y - exp)) < 1e-3


def c2psa_fixture():
    fam = "c2psa_yolo26"
    P = Y.Params(block_params(fam, _shapes(fam, {"m.0.attn.pe": 3})), eps=EPS_FIXTURE)
    x = load(f"{fam}/x.bin", (2, 256, 4, 4))
    exp = load(f"{fam}/expected_output.bin", (2, 256, 4, 4))
    return P, x, exp


def test_c2psa():
    P, x, exp = c2psa_fixture()
    y = Y.c2psa(256, 256, 1, 0.5)(P, "", x)
    assert np.max(np.abs(y - exp)) < 1e-3


def test_psa_attention_core_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    B, heads, kd, vd, H, W = 2, 3, 32, 64, 5, 7
    qkv = rng.standard_normal((B, heads * (2 * kd + vd), H, W)).astype(np.float32)
    out = oracle.psa_attention(qkv, heads, kd, vd)
    t = torch.from_numpy(qkv).view(B, heads, 2 * kd + vd, H * W)
    q, k, v = t.split([kd, kd, vd], dim=2)
    a = ((q.transpose(-2, -1) @ k) * kd ** -0.5).softmax(-1)
    ref = (v @ a.transpose(-2, -1)).reshape(B, heads * vd, H, W).numpy()
    assert np.allclose(out, ref, rtol=1e-4, atol=1e-5)


def sppf_fixture():
    fam = "sppf_yolo26"
    P = Y.Params(block_params(fam, _shapes(fam, {})), eps=EPS_FIXTURE)
    x = load(f"{fam}/x.bin", (2, 32, 4, 4))
    exp = load(f"{fam}/expected_output.bin", (2, 32, 4, 4))
    return P, x, exp


def test_sppf():
    P, x, exp = sppf_fixture()
    # ultralytics SPPF default shortcut=False (tests/fixtures/sppf_yolo26/generate.py)
    y = Y.sppf(32, 32, False)(P, "", x)
    assert np.max(np.abs(y - exp)) < 1e-3


def detect_fixture():
    fam = "detect_yolo26"
    P = Y.Params(eps=EPS_FIXTURE)
    for i, (co, ci, k) in enumerate([(64, 256, 3), (64, 64, 3)], start=1):
        P[f"{i - 1}.conv.weight"] = load(f"{fam}/conv{i}_w.bin", (co, ci, k, k))
        for a, b in (("w", "weight"), ("b", "bias"), ("rm", "running_mean"), ("rv", "running_var")):
            P[f"{i - 1}.bn.{b}"] = load(f"{fam}/conv{i}_bn_{a}.bin")
    P["2.weight"] = load(f"{fam}/conv3_w.bin", (4, 64, 1, 1))
    P["2.bias"] = load(f"{fam}/conv3_bias.bin")
    x = load(f"{fam}/x.bin", (1, 256, 4, 4))
    exp = load(f"{fam}/expected_output.bin", (1, 4, 4, 4))
    return P, x, exp


def test_detect_box_branch():
    P, x, exp = detect_fixture()
    y = Y.conv(256, 64, 3, 1)(P, "0", x)
    y = Y.conv(64, 64, 3, 1)(P, "1", y)
    y = Y.conv_plain(64, 4, 1, 1)(P, "2", y)
    assert np.max(np.abs(y - exp)) < 1e-3


# ------------------------------------------------------------ post-process --

def test_detect_decode_grid_fixture():
    B, A = 2, 16
    boxes = load("detect_decode/raw_boxes.bin", (B, 4, A))
    out = oracle.detect_decode_grid(boxes, load("detect_decode/anchor_x.bin"),
                                    load("detect_decode/anchor_y.bin"), load("detect_decode/strides.bin"))
    assert np.max(np.abs(out - load("detect_decode/expected.bin", (B, 4, A)))) < 1e-4


def _brute_postprocess(boxes, scores, nc, img, strides, thr, max_det):
    """Pure-Python restatement of examples/yolo26.rs:1488-1529 for small inputs."""
    import math
    out = []
    for b in range(boxes.shape[0]):
        cands, base = [], 0
        for s in strides:
            fw, fh = img // s, img // s
            a_s = fw * fh
            bb = boxes[b, 4 * base: 4 * (base + a_s)].reshape(4, a_s)
            ss = scores[b, nc * base: nc * (base + a_s)].reshape(nc, a_s)
            for j in range(a_s):
                best, bc = None, None
                for c in range(nc):
                    v = np.float32(1.0) / (np.float32(1.0) + np.float32(math.exp(-float(ss[c, j]))))
                    if best is None or not (best > v):
                        best, bc = v, c
                if best >= thr:
                    cands.append((float(best), bc, base + j))
            base += a_s
        cands.sort(key=lambda t: -t[0])  # stable
        out.append(cands[:max_det])
    return out


def test_detect_postprocess_brute_force_and_ties():
    rng = np.random.default_rng(4)
    nc, img, strides = 5, 64, (8, 16, 32)
    A = sum((img // s) ** 2 for s in strides)
    B = 2
    boxes = rng.uniform(0, 4, (B, 4 * A)).astype(np.float32)
    scores = rng.normal(0, 2, (B, nc * A)).astype(np.float32)
    # plant exact ties: equal logits in two classes (last class must win) and
    # equal best scores across anchors (ascending anchor order must be kept)
    scores[0, 0 * 64 + 3] = 3.0; scores[0, 1 * 64 + 3] = 3.0; scores[0, 4 * 64 + 3] = 3.0
    scores[0, 2 * 64 + 10] = 3.0
    count, sc, cl, an, xy = oracle.detect_postprocess(boxes, scores, nc, img, img, strides, 0.25, 50)
    ref = _brute_postprocess(boxes, scores, nc, img, strides, 0.25, 50)
    for b in range(B):
        assert count[b] == len(ref[b])
        for i, (s, c, a) in enumerate(ref[b]):
            assert sc[b, i] == np.float32(s) and cl[b, i] == c and an[b, i] == a
    i3 = list(an[0]).index(3)
    assert cl[0, i3] == 4  # last of the tied classes wins
    # closed-form decode for anchor 0 of scale 8: centre (4, 4)
    a0 = list(an[0]).index(an[0][0])
    a = an[0][a0]
    if a < 64:
        l, t, r, bo = boxes[0, a], boxes[0, 64 + a], boxes[0, 128 + a], boxes[0, 192 + a]
        cx = ((a % 8) + 0.5) * 8; cy = ((a // 8) + 0.5) * 8
        assert np.allclose(xy[0, a0], [cx + 8 * (r - l) * 0.5, cy + 8 * (bo - t) * 0.5, 8 * (l + r), 8 * (t + bo)])


# -------------------------------------------------------------------- MSDA --

def _msda_torch(value, shapes, ref, off, attw):
    """Deformable-DETR multi_scale_deformable_attn_pytorch formulation via grid_sample."""
    import torch
    import torch.nn.functional as F
    v = torch.from_numpy(value)
    B, S, h, Dh = v.shape
    _, Q, _, L, P, _ = off.shape
    loc = torch.from_numpy(ref)[:, :, None, None, None, :] + torch.from_numpy(off)
    grids = 2 * loc - 1
    out = 0
    start = 0
    for l, (H, W) in enumerate(shapes):
        vl = v[:, start:start + H * W].permute(0, 2, 3, 1).reshape(B * h, Dh, H, W)
        g = grids[:, :, :, l].permute(0, 2, 1, 3, 4).reshape(B * h, Q, P, 2)
        s = F.grid_sample(vl, g, mode="bilinear", padding_mode="zeros", align_corners=False)  # [Bh,Dh,Q,P]
        a = torch.from_numpy(attw)[:, :, :, l].permute(0, 2, 1, 3).reshape(B * h, 1, Q, P)
        out = out + (s * a).sum(-1)
        start += H * W
    return out.view(B, h * Dh, Q).transpose(1, 2).contiguous().numpy()


def msda_inputs(B, Q, heads, Dh, shapes, P, seed=5):
    rng = np.random.default_rng(seed)
    S = sum(h * w for h, w in shapes)
    L = len(shapes)
    value = rng.standard_normal((B, S, heads, Dh)).astype(np.float32)
    ref = rng.uniform(0, 1, (B, Q, 2)).astype(np.float32)
    off = rng.normal(0, 0.05, (B, Q, heads, L, P, 2)).astype(np.float32)
    logits = rng.standard_normal((B, Q, heads, L * P)).astype(np.float32)
    e = np.exp(logits - logits.max(-1, keepdims=True))
    attw = (e / e.sum(-1, keepdims=True)).reshape(B, Q, heads, L, P).astype(np.float32)
    return value, ref, off, attw


def test_detect_unletterbox_closed_forms():
    """Un-letterbox (examples/yolo26.rs:1531-1547) pinned by cases whose
    scale and padding are known exactly: a square image (divide by its side),
    2:1 landscape / portrait (scale 1/2, 140-pixel bars), a size whose scaled
    side rounds (333x777 -> 274 wide, 183-pixel bars), and zeroed slots."""
    xywh = np.zeros((5, 3, 4), np.float32)
    xywh[0, 0] = (160, 480, 320, 64)      # 640x640 -> divide by 640
    xywh[1, 0] = (320, 320, 640, 360)     # 1280x720 letterboxed: the whole image
    xywh[1, 1] = (0, 140, 64, 36)         # its top-left corner
    xywh[2, 0] = (320, 320, 360, 640)     # 720x1280
    xywh[3, 0] = (183, 320, 0, 640)       # 333x777: left bar ends at x = 183
    xywh[4, 0] = (1, 2, 3, 4)             # count 0: zeroed
    wh = np.array([[640, 640], [1280, 720], [720, 1280], [333, 777], [10, 10]], np.int32)
    count = np.array([1, 2, 1, 1, 0], np.int32)
    out = oracle.detect_unletterbox(count, xywh, wh, 640)
    assert out[0, 0].tolist() == [0.25, 0.75, 0.5, np.float32(0.1)]
    assert out[1, 0].tolist() == [0.5, 0.5, 1.0, 1.0]
    assert out[1, 1].tolist() == [0.0, 0.0, np.float32(0.1), np.float32(0.1)]
    assert out[2, 0].tolist() == [0.5, 0.5, 1.0, 1.0]
    assert out[3, 0][0] == 0.0 and out[3, 0][2] == 0.0   # pad_x = (640 - 274) // 2 = 183
    assert out[3, 0][3] == np.float32(640) / np.float32(np.float32(777) * (np.float32(640) / np.float32(777)))
    assert not out[0, 1:].any() and not out[1, 2:].any() and not out[4].any()


LETTERBOX_SIZES = [(1280, 720, 640), (517, 333, 640), (333, 517, 640), (1000, 37, 640), (5, 3, 640),
                   (4000, 100, 64), (17, 2000, 640), (8, 8, 4), (2, 1, 4), (640, 640, 640), (1, 1, 32)]


@pytest.mark.parametrize("w,h,S", LETTERBOX_SIZES)
def test_letterbox_resize_matches_torch_antialias(w, h, S):
    """The Triangle resize (image 0.25.10, restated in orc_letterbox) against
    torch's antialiased bilinear interpolation, an independent implementation
    (PIL's formulation) of the same filter: tent of support max(ratio, 1)
    centred at (o + 0.5) * ratio, weights normalised over the clamped window.
    Compared on the float stage before u8 rounding."""
    torch = pytest.importorskip("torch")
    img = np.random.default_rng(w * 7 + h).integers(0, 256, (h, w, 3), dtype=np.uint8)
    out, res = oracle.letterbox(img, S, resized=True)
    nh, nw, _ = res.shape
    ref = torch.nn.functional.interpolate(torch.from_numpy(img).permute(2, 0, 1)[None].float(), size=(nh, nw),
                                          mode="bilinear", antialias=True, align_corners=False)
    ref = ref[0].permute(1, 2, 0).numpy()
    assert np.abs(ref - res).max() < 2e-4
    # the canvas holds round-half-away(clamp(res)) / 255 at the centred offset
    px, py = (S - nw) // 2, (S - nh) // 2
    q = (np.floor(np.clip(res, 0, 255) + 0.5) / np.float32(255)).astype(np.float32)
    assert np.array_equal(out[:, py:py + nh, px:px + nw], q.transpose(2, 0, 1))
    pad = np.ones((S, S), bool)
    pad[py:py + nh, px:px + nw] = False
    assert (out[:, pad] == np.float32(114) / np.float32(255)).all()


def test_letterbox_closed_forms():
    """Geometry of preprocess_image_raw (examples/yolo26.rs:1229-1253) and the
    Triangle filter's exact cases: same size is the identity, a 2x shrink
    weights interior taps [1, 3, 3, 1] / 8 per axis, and a 2x enlargement
    interpolates at 1/4 and 3/4 with half-way values rounded away from zero."""
    rng = np.random.default_rng(5)
    # geometry: new size rounds in f64, padding is integer-halved
    for (w, h, nw, nh) in [(1280, 720, 640, 360), (333, 517, 412, 640), (1000, 37, 640, 24), (17, 2000, 5, 640)]:
        _, res = oracle.letterbox(np.zeros((h, w, 3), np.uint8), 640, resized=True)
        assert res.shape == (nh, nw, 3)
    # identity
    img = rng.integers(0, 256, (640, 640, 3), dtype=np.uint8)
    out = oracle.letterbox(img, 640)
    assert np.array_equal(out, (img.astype(np.float32) / np.float32(255)).transpose(2, 0, 1))
    # 2x shrink: 8x8 -> 4x4, output (1, 1) reads rows/cols 1..4 with [1,3,3,1]/8
    img = rng.integers(0, 256, (8, 8, 3), dtype=np.uint8)
    _, res = oracle.letterbox(img, 4, resized=True)
    k = np.array([1, 3, 3, 1], np.float64) / 8
    for c in range(3):
        for oy, ox in [(1, 1), (1, 2), (2, 1), (2, 2)]:
            win = img[2 * oy - 1:2 * oy + 3, 2 * ox - 1:2 * ox + 3, c].astype(np.float64)
            assert abs(res[oy, ox, c] - k @ win @ k) < 1e-4
    # 2x enlargement of the 2x1 row [0, 2]: [0, 0.5, 1.5, 2] -> u8 [0, 1, 2, 2]
    img = np.zeros((1, 2, 3), np.uint8)
    img[0, 1] = 2
    out, res = oracle.letterbox(img, 4, resized=True)
    assert res[:, :, 0].tolist() == [[0, 0.5, 1.5, 2]] * 2
    pad = np.float32(114) / np.float32(255)
    assert out[0].tolist() == [[pad] * 4, [0, np.float32(1) / 255, np.float32(2) / 255, np.float32(2) / 255],
                               [0, np.float32(1) / 255, np.float32(2) / 255, np.float32(2) / 255], [pad] * 4]


def test_msda_matches_grid_sample():
    pytest.importorskip("torch")
    shapes = [(16, 16), (8, 8), (4, 4), (2, 2)]
    value, ref, off, attw = msda_inputs(2, 30, 4, 32, shapes, 4)
    out = oracle.msda(value, shapes, ref, off, attw)
    assert np.allclose(out, _msda_torch(value, shapes, ref, off, attw), rtol=1e-4, atol=1e-5)


def test_msda_brute_tiny():
    # one head, one level, one point; a sample exactly on pixel centre (i, j)
    # returns value[i, j]; half a pixel outside the map gives half weight.
    H, W = 4, 5
    value = np.arange(H * W, dtype=np.float32).reshape(1, H * W, 1, 1)
    ref = np.array([[[(2 + 0.5) / W, (1 + 0.5) / H]]], np.float32)
    off = np.zeros((1, 1, 1, 1, 1, 2), np.float32)
    attw = np.ones((1, 1, 1, 1, 1), np.float32)
    assert oracle.msda(value, [(H, W)], ref, off, attw)[0, 0, 0] == value[0, 1 * W + 2, 0, 0]
    ref = np.array([[[0.0, (1 + 0.5) / H]]], np.float32)  # x = -0.5 px: half of column 0
    assert abs(oracle.msda(value, [(H, W)], ref, off, attw)[0, 0, 0] - 0.5 * value[0, W, 0, 0]) < 1e-6


def test_e4m3_round_matches_torch():
    """Pins oracle.yolo26.e4m3_round (the fp8 emulation) to torch's OCP e4m3
    conversion: ties to even, subnormals, the 448 maximum; values beyond 448
    saturate (the device clamps before converting)."""
    import torch
    from oracle.yolo26 import e4m3_round
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100000) * np.exp(rng.uniform(-12, 7, 100000))
    edges = [448, -448, 0.0, 2 ** -9, 2 ** -10, 3 * 2 ** -10, 2 ** -6, 1.0625, 1.1875, 232, 240, 464 - 1e-3]
    x = np.concatenate([x, edges]).astype(np.float32)
    x = x[np.abs(x) <= 448]
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(e4m3_round(x), ref)
    assert np.array_equal(e4m3_round(np.array([500.0, -1e6, 449.0], np.float32)), np.array([448, -448, 448.0]))

