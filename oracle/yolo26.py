"""CPU restatement of the YOLO26 layer wiring (TEST INFRASTRUCTURE ONLY).

Mirrors the reference's closure builders one for one; each builder returns a
callable ``f(P, pre, x)`` where ``P`` maps parameter names to float32 arrays
and ``pre`` is the name_scope prefix (reference names, e.g.
``model.6.m.0.m.1.cv2.conv.weight``).  Tensors are NCHW float32 numpy arrays.

Reference anchors:
  conv / conv_bn / dwconv / conv_plain     blocks/conv.rs:31-99
  bottleneck_std / bottleneck_3x3          blocks/bottleneck.rs:37-63
  c3k_inner / c3k2 / c3k2_psa              blocks/c3k2.rs:46-164
  psa_attention / psa_block / c2psa        blocks/c2psa.rs:61-179
  sppf                                     blocks/sppf.rs:43-61
  upsample / concat                        blocks/upsample.rs:23-35, blocks/concat.rs:24-38
  detect (+ channel_cat_flat)              blocks/detect.rs:62-172
  variant config, ch, rep, build_neck      yolo26/mod.rs:57-195
  yolo26                                   yolo26/mod.rs:207-219
"""
from __future__ import annotations

import math

import numpy as np

from . import affine_act, bn_fold, conv2d, maxpool2d, psa_attention, upsample_nearest

SILU, NONE = 1, 0

VARIANTS = {  # yolo26/mod.rs:70-100 (depth, width, max_channels)
    "n": (0.5, 0.25, 1024),
    "s": (0.5, 0.50, 1024),
    "m": (0.5, 1.00, 512),
    "l": (1.0, 1.00, 512),
    "x": (1.0, 1.50, 512),
}


def _round(v: float) -> int:  # Rust f32::round: half away from zero
    return int(math.floor(v + 0.5))


def ch(base, width, mc):  # mod.rs:106-108
    return _round(min(base, mc) * width)


def rep(base, depth):  # mod.rs:111-117
    return _round(max(base * depth, 1.0)) if base > 1 else base


def _j(pre, name):
    return f"{pre}.{name}" if pre else name


class Params(dict):
    """Name -> array, plus the BN eps the model folds with (1e-3 in the model,
    blocks/conv.rs:39; 1e-5 for the reference's PyTorch-made fixtures).

    ``act_q`` (identity by default) is applied wherever an activation tensor is
    materialised -- each conv output (after its residual add, which belongs to
    the same elem_add node of the reference graph) and the attention output --
    so a bfloat16 run can be compared against an oracle that stores its
    activations at the same precision and at the same points."""

    def __init__(self, *a, eps=1e-3, act_q=None, fp8=None, observe=None, store8=None, **k):
        super().__init__(*a, **k)
        self.eps = eps
        self.act_q = act_q if act_q is not None else (lambda t: t)
        # conv prefix -> activation step of the convs that run on e4m3
        # (weights per output channel, inputs per tensor; see fp8_conv_inputs)
        self.fp8 = fp8 or {}
        # conv prefix -> step of the convs whose output is stored as e4m3: the
        # stored value is e4m3(act_q(y) / step) * step
        self.store8 = store8 or {}
        # observe(prefix, x): called with every dense/depthwise conv's input
        # before the conv (fp8_steps records max |x| through it)
        self.observe = observe


def e4m3_round(x):
    """float32 -> nearest OCP e4m3 value (ties to even, saturating at +-448,
    subnormal step 2^-9).  No reference function (BASELINE config 5's fp8
    run); pinned against torch.float8_e4m3fn in tests/test_oracle_golden.py."""
    x = np.asarray(x, np.float32)
    a = np.minimum(np.abs(x), np.float32(448.0))
    sub = np.rint(a * np.float32(512.0)) / np.float32(512.0)
    f, e2 = np.frexp(np.maximum(a, np.float32(2.0 ** -6)))
    mant = np.rint((f * 2.0 - 1.0) * 8.0).astype(np.float32)
    norm = np.ldexp(np.float32(1.0) + mant / np.float32(8.0), e2 - 1).astype(np.float32)
    return np.where(a < 2.0 ** -6, sub, norm).astype(np.float32) * np.sign(x).astype(np.float32)


def fp8_conv_inputs(x, w, in_scale):
    """The e4m3 operands of an fp8 conv, dequantised: x on the per-tensor step
    in_scale (a power of two), w per output channel on step max|w|/448."""
    wf = np.asarray(w, np.float32)
    amax = np.abs(wf.reshape(wf.shape[0], -1)).max(axis=1).astype(np.float32)
    sc = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    scb = sc.reshape(-1, *([1] * (wf.ndim - 1)))
    wq = e4m3_round(wf / scb) * scb
    s = np.float32(in_scale)
    return e4m3_round(np.asarray(x, np.float32) / s) * s, wq.astype(np.float32)


def fp8_step(amax):
    """Activation step of an fp8 conv input as vrs_model_calibrate sets it:
    the smallest power of two >= amax / 448 (1 for an all-zero input)."""
    if not amax > 0 or not np.isfinite(amax):
        return 1.0
    f, e = math.frexp(float(np.float32(amax) / np.float32(448.0)))
    return math.ldexp(1.0, e - 1 if f == 0.5 else e)


def fp8_steps(net, P, x, prefixes):
    """{prefix: step} for the convs in `prefixes` from one forward of `net`
    (e.g. yolo26(...)) on x with P (its act_q sets the activation precision
    of the calibrating forward): the per-tensor max |input| of each conv."""
    amax = {}

    def see(pre, t):
        if pre in prefixes:
            amax[pre] = max(amax.get(pre, 0.0), float(np.max(np.abs(t))))
    Q = Params(P, eps=P.eps, act_q=P.act_q, observe=see, store8=P.store8)
    net(Q, x)
    return {pre: fp8_step(a) for pre, a in amax.items()}


def _conv_bn_act(P, pre, x, k, s, g, act, res=None):
    w = P[_j(pre, "conv.weight")]
    if P.observe is not None:
        P.observe(pre, x)
    if pre in P.fp8:
        x, w = fp8_conv_inputs(x, w, P.fp8[pre])
    y = conv2d(x, w, stride=s, pad=k // 2, groups=g)
    scale, shift = bn_fold(P[_j(pre, "bn.weight")], P[_j(pre, "bn.bias")],
                           P[_j(pre, "bn.running_mean")], P[_j(pre, "bn.running_var")], P.eps)
    y = affine_act(y, scale, shift, act)
    if res is not None:  # elem_add(x, conv(...)) of the caller (bottleneck.rs:24-30)
        y = y + res
    y = P.act_q(y)
    if pre in P.store8:
        st = np.float32(P.store8[pre])
        y = e4m3_round(y / st) * st
    return y


def conv(c_in, c_out, k, s):  # conv.rs:31-46: Conv2d(no bias, pad k/2) -> BN -> SiLU
    return lambda P, pre, x, res=None: _conv_bn_act(P, pre, x, k, s, 1, SILU, res)


def conv_bn(c_in, c_out, k, s, g):  # conv.rs:53-69: grouped conv -> BN, no act
    return lambda P, pre, x, res=None: _conv_bn_act(P, pre, x, k, s, g, NONE, res)


def dwconv(c, k, s):  # conv.rs:75-85: depthwise -> BN -> SiLU
    return lambda P, pre, x: _conv_bn_act(P, pre, x, k, s, c, SILU)


def conv_plain(c_in, c_out, k, s):  # conv.rs:90-99: conv with bias
    def f(P, pre, x):
        w = P[_j(pre, "weight")]
        if P.observe is not None:
            P.observe(pre, x)
        if pre in P.fp8:
            x, w = fp8_conv_inputs(x, w, P.fp8[pre])
        return conv2d(x, w, stride=s, pad=k // 2, bias=P[_j(pre, "bias")])
    return f


def bottleneck_std(c, shortcut):  # bottleneck.rs:37-49: shortcut -> elem_add(x, y)
    ci = int(c * 0.5)
    cv1, cv2 = conv(c, ci, 3, 1), conv(ci, c, 3, 1)
    return lambda P, pre, x: cv2(P, _j(pre, "cv2"), cv1(P, _j(pre, "cv1"), x), x if shortcut else None)


def bottleneck_3x3(c, shortcut):  # bottleneck.rs:51-63
    cv1, cv2 = conv(c, c, 3, 1), conv(c, c, 3, 1)
    return lambda P, pre, x: cv2(P, _j(pre, "cv2"), cv1(P, _j(pre, "cv1"), x), x if shortcut else None)


def c3k_inner(c, shortcut):  # c3k2.rs:46-61
    ch_ = int(c * 0.5)
    cv1, cv2, cv3 = conv(c, ch_, 1, 1), conv(c, ch_, 1, 1), conv(2 * ch_, c, 1, 1)
    m0, m1 = bottleneck_3x3(ch_, shortcut), bottleneck_3x3(ch_, shortcut)

    def f(P, pre, x):
        a = cv1(P, _j(pre, "cv1"), x)
        a = m0(P, _j(pre, "m.0"), a)
        a = m1(P, _j(pre, "m.1"), a)
        b = cv2(P, _j(pre, "cv2"), x)
        return cv3(P, _j(pre, "cv3"), np.concatenate([a, b], axis=1))
    return f


def _c2f(cv1, cv2, blocks, c):
    def f(P, pre, x):  # c3k2.rs:113-126
        h = cv1(P, _j(pre, "cv1"), x)
        parts = [h[:, :c], h[:, c:2 * c]]
        last = parts[1]
        for i, b in enumerate(blocks):
            last = b(P, _j(pre, f"m.{i}"), last)
            parts.append(last)
        return cv2(P, _j(pre, "cv2"), np.concatenate(parts, axis=1))
    return f


def c3k2(c_in, c_out, n, c3k, shortcut, e):  # c3k2.rs:94-127
    c = int(c_out * e)
    blocks = [c3k_inner(c, shortcut) if c3k else bottleneck_std(c, shortcut) for _ in range(n)]
    return _c2f(conv(c_in, 2 * c, 1, 1), conv((2 + n) * c, c_out, 1, 1), blocks, c)


def psa_attention_block(c, num_heads, key_dim):  # c2psa.rs:61-116
    head_dim = c // num_heads
    qkv_h = num_heads * (2 * key_dim + head_dim)
    qkv = conv_bn(c, qkv_h, 1, 1, 1)
    proj = conv_bn(c, c, 1, 1, 1)

    def f(P, pre, x, res=None):
        B, _, H, W = x.shape
        q = qkv(P, _j(pre, "qkv"), x)
        att = psa_attention(q, num_heads, key_dim, head_dim)
        # V channels per head -> [B, c, H, W] (psa.rs:104-142); PE conv_bn on V
        v = q.reshape(B, num_heads, 2 * key_dim + head_dim, H, W)[:, :, 2 * key_dim:]
        v = np.ascontiguousarray(v.reshape(B, c, H, W))
        w = P[_j(pre, "pe.conv.weight")]
        scale, shift = bn_fold(P[_j(pre, "pe.bn.weight")], P[_j(pre, "pe.bn.bias")],
                               P[_j(pre, "pe.bn.running_mean")], P[_j(pre, "pe.bn.running_var")], P.eps)
        pe_out = affine_act(conv2d(v, w, stride=1, pad=1, groups=c), scale, shift, NONE)
        return proj(P, _j(pre, "proj"), P.act_q(att + pe_out), res)  # elem_add(merged, pe) (:112)
    return f


def psa_block(c, num_heads, key_dim):  # c2psa.rs:123-137: b += attn(b); b += ffn(b)
    attn = psa_attention_block(c, num_heads, key_dim)
    ffn0, ffn1 = conv(c, 2 * c, 1, 1), conv_bn(2 * c, c, 1, 1, 1)

    def f(P, pre, b):
        b = attn(P, _j(pre, "attn"), b, b)
        return ffn1(P, _j(pre, "ffn.1"), ffn0(P, _j(pre, "ffn.0"), b), b)
    return f


def c2psa(c_in, c_out, n, e):  # c2psa.rs:150-179
    assert c_in == c_out
    c = int(c_out * e)
    cv1, cv2 = conv(c_in, 2 * c, 1, 1), conv(2 * c, c_out, 1, 1)
    blocks = [psa_block(c, c // 64, 32) for _ in range(n)]

    def f(P, pre, x):
        h = cv1(P, _j(pre, "cv1"), x)
        a, b = h[:, :c], h[:, c:]
        for i, blk in enumerate(blocks):
            b = blk(P, _j(pre, f"m.{i}"), b)
        return cv2(P, _j(pre, "cv2"), np.concatenate([a, b], axis=1))
    return f


def c3k2_psa(c_in, c_out, n, shortcut, e):  # c3k2.rs:134-164 (+ bottleneck_psa_seq :67-79)
    c = int(c_out * e)
    heads, kd = c // 64, 32

    def seq():
        bn, ps = bottleneck_std(c, shortcut), psa_block(c, heads, kd)
        return lambda P, pre, x: ps(P, _j(pre, "1"), bn(P, _j(pre, "0"), x))
    return _c2f(conv(c_in, 2 * c, 1, 1), conv((2 + n) * c, c_out, 1, 1), [seq() for _ in range(n)], c)


def sppf(c_in, c_out, shortcut):  # sppf.rs:43-61
    c = c_in // 2
    add = shortcut and c_in == c_out
    cv1, cv2 = conv_bn(c_in, c, 1, 1, 1), conv(4 * c, c_out, 1, 1)

    def f(P, pre, x):
        y = cv1(P, _j(pre, "cv1"), x)
        p1 = maxpool2d(y); p2 = maxpool2d(p1); p3 = maxpool2d(p2)
        return cv2(P, _j(pre, "cv2"), np.concatenate([y, p1, p2, p3], axis=1), x if add else None)
    return f


def detect(nc, chs, one2one=True):  # detect.rs:108-172 (reg_max = 1)
    c2 = max(16, chs[0] // 4, 4)
    c3 = max(chs[0], min(nc, 100))
    p2, p3 = ("one2one_cv2", "one2one_cv3") if one2one else ("cv2", "cv3")
    box = [(conv(ci, c2, 3, 1), conv(c2, c2, 3, 1), conv_plain(c2, 4, 1, 1)) for ci in chs]
    cls = [(dwconv(ci, 3, 1), conv(ci, c3, 1, 1), dwconv(c3, 3, 1), conv(c3, c3, 1, 1),
            conv_plain(c3, nc, 1, 1)) for ci in chs]

    def f(P, pre, feats):
        bx, sc = [], []
        for i, x in enumerate(feats):
            q = _j(pre, f"{p2}.{i}")
            y = box[i][0](P, _j(q, "0"), x)
            y = box[i][1](P, _j(q, "1"), y)
            bx.append(box[i][2](P, _j(q, "2"), y))
        for i, x in enumerate(feats):
            q = _j(pre, f"{p3}.{i}")
            y = cls[i][0](P, _j(q, "0.0"), x)
            y = cls[i][1](P, _j(q, "0.1"), y)
            y = cls[i][2](P, _j(q, "1.0"), y)
            y = cls[i][3](P, _j(q, "1.1"), y)
            sc.append(cls[i][4](P, _j(q, "2"), y))
        B = feats[0].shape[0]
        # channel_cat_flat (detect.rs:62-80): per scale, NCHW flattened
        boxes = np.concatenate([t.reshape(B, -1) for t in bx], axis=1)
        scores = np.concatenate([t.reshape(B, -1) for t in sc], axis=1)
        return boxes, scores
    return f


def build_neck(variant):  # mod.rs:126-195
    d, w, mc = VARIANTS[variant]
    c0, c1, c2, c3, c4 = (ch(b, w, mc) for b in (64, 128, 256, 512, 1024))
    n = rep(2, d)
    L = {
        0: conv(3, c0, 3, 2), 1: conv(c0, c1, 3, 2), 2: c3k2(c1, c2, n, False, True, 0.25),
        3: conv(c2, c2, 3, 2), 4: c3k2(c2, c3, n, False, True, 0.25), 5: conv(c3, c3, 3, 2),
        6: c3k2(c3, c3, n, True, True, 0.5), 7: conv(c3, c4, 3, 2), 8: c3k2(c4, c4, n, True, True, 0.5),
        9: sppf(c4, c4, True), 10: c2psa(c4, c4, n, 0.5),
        13: c3k2(c4 + c3, c3, n, True, True, 0.5), 16: c3k2(c3 + c3, c2, n, True, True, 0.5),
        17: conv(c2, c2, 3, 2), 19: c3k2(c2 + c3, c3, n, True, True, 0.5), 20: conv(c3, c3, 3, 2),
        22: c3k2_psa(c3 + c4, c4, 1, True, 0.5),
    }

    def neck(P, x):
        m = lambda i, t: L[i](P, f"model.{i}", t)  # noqa: E731
        x = m(0, x); x = m(1, x); x = m(2, x); x = m(3, x)
        p3 = m(4, x)
        x = m(5, p3); p4 = m(6, x)
        x = m(7, p4); x = m(8, x); x = m(9, x); p5 = m(10, x)
        x = np.concatenate([upsample_nearest(p5), p4], axis=1)
        nk4 = m(13, x)
        x = np.concatenate([upsample_nearest(nk4), p3], axis=1)
        p3d = m(16, x)
        x = np.concatenate([m(17, p3d), nk4], axis=1)
        p4d = m(19, x)
        x = np.concatenate([m(20, p4d), p5], axis=1)
        p5d = m(22, x)
        return p3d, p4d, p5d

    return neck, (c2, c3, c4)


def yolo26(nc, variant, one2one=True):  # mod.rs:207-219
    neck, chs = build_neck(variant)
    head = detect(nc, list(chs), one2one)

    def f(P, x):
        return head(P, "model.23", list(neck(P, x)))
    return f
