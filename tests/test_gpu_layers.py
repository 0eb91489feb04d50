"""Layer by layer (teacher-forced) parity of the whole YOLO26m network at
BASELINE config 5's full size (batch 64, 640x640), bf16 and fp8.

The forward runs the committed tile plans (the bench line's kernels) and is
replayed one kernel launch at a time (a fused pair -- the stem pair, a
bottleneck pair -- is one launch: its second conv is checked on the first
conv's output recomputed by the oracle).  Before each conv's
launch its actual device input (and residual, and the half-size source of a
fused upsample) is read back for images 0 and 31; after it, its output.  The
oracle then recomputes that one conv from the device's own input, so every
layer is held to the single-kernel bar -- elementwise 2e-2 relative with a
floor of 0.1 * rms (test_gpu_ops) -- with no drift carried in from earlier
layers:

* bf16: the oracle conv on the same bf16 operands;
* fp8 (every eligible conv forced onto the e4m3 MFMA, as the bench's forced
  fp8 line runs): the oracle conv on the same dequantised e4m3 operands --
  the input quantised with the layer's calibrated power-of-two step, the
  weights per output channel on max|w|/448 (the fp8 configuration's CPU
  check uses the same dequantised weights and activation scales).

The end-to-end outputs of the same run are then compared with the plain
float32 oracle (the reference CPU path on the unrounded weights and input):

* bf16: normwise error < 2e-2; identical class argmax wherever the float32
  top-2 logit margin exceeds twice the tolerance, 2 * 2e-2 * std(logits) (two
  logits each within 2e-2 of the logits' spread cannot trade places); the
  device post-process's top-k anchors identical to the oracle's at every rank
  whose float32 best-class logit is separated from both neighbours' by that
  margin.
* fp8: an e4m3 activation carries 3 mantissa bits, and one-ulp differences of
  the bf16 values it is rounded from (the device and the oracle sum in
  different orders) flip e4m3 roundings that compound over ~90 layers
  (tests/test_fp8_sensitivity.py shows this on the oracle alone: 0.1 % of
  activations moved by one bf16 ulp move the e4m3 emulation by 7.5e-2 /
  9.3e-2).  No fp8 pipeline meets 2e-2 of float32 here; the stated fp8 bar is
  normwise < 0.15 against float32 (the emulation itself is at 0.104 / 0.126)
  and < 0.13 against the precision-matched emulation, and the device no
  farther from float32 than 1.2x the emulation is.  Per layer, fp8 is held to
  the same 2e-2 single-kernel bar as bf16 (above).
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from oracle import yolo26 as Y
from gpu_util import bf16_round, ctx, dev, rel_err, vrs
from test_gpu_ops import e4m3_bracket
from golden_io import seeded_params

pytestmark = pytest.mark.gpu

IMAGES = (0, 31)
_hip = None


def _d2h(ptr, nbytes):
    """Device -> host copy of raw model memory (synchronous hipMemcpy)."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip.hipMemcpy.restype = C.c_int
    out = np.empty(nbytes, np.uint8)
    rc = _hip.hipMemcpy(out.ctypes.data, C.c_void_p(ptr), nbytes, 2)   # hipMemcpyDeviceToHost
    assert rc == 0, rc
    return out


_E4M3 = None


def e4m3_values():
    """float32 value of each e4m3 byte (OCP E4M3FN, as torch.float8_e4m3fn)."""
    global _E4M3
    if _E4M3 is None:
        import torch
        _E4M3 = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    return _E4M3


def read_view(v, dtype, images, e4m3=False, step=0.0):
    """NCHW float32 [len(images), c, h, w] of an NHWC view of model memory
    (e4m3: a view of a buffer stored as e4m3 bytes on `step`)."""
    es = 1 if e4m3 else 4 if dtype == vrs.F32 else 2
    per = v.h * v.w * v.pitch * es
    out = []
    for i in images:
        raw = _d2h(v.data + i * per, per)
        if e4m3:
            a = e4m3_values()[raw] * np.float32(step)
        elif es == 2:
            a = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        else:
            a = raw.view(np.float32)
        a = a.reshape(v.h, v.w, v.pitch)[:, :, v.c_off:v.c_off + v.c]
        out.append(a.transpose(2, 0, 1))
    return np.ascontiguousarray(np.stack(out))


def read_flat(io, outs, images, ho, wo):
    """A conv's float32 output inside model output io.out_idx (flat layout)."""
    o = outs[io.out_idx].cpu().numpy().reshape(-1)
    p = np.arange(ho * wo)
    c = np.arange(io.cout)
    res = []
    for i in images:
        idx = io.out_off + i * io.out_sb + c[:, None] * io.out_sc + p[None, :] * io.out_sp
        res.append(o[idx].reshape(io.cout, ho, wo))
    return np.stack(res)


def conv_reference(io, P, eps, x, res):
    """The oracle conv of one layer on the layer's own input x (NCHW f32)."""
    pre = io.prefix
    w = P[f"{pre}.weight"] if io.plain else P[f"{pre}.conv.weight"]
    if io.fp8:
        x, w = Y.fp8_conv_inputs(x, w, io.in_scale)
    y = oracle.conv2d(x, w, io.stride, io.k // 2, groups=io.groups)
    if io.plain:
        y = y + P[f"{pre}.bias"].reshape(1, -1, 1, 1)
    else:
        scale, shift = oracle.bn_fold(P[f"{pre}.bn.weight"], P[f"{pre}.bn.bias"], P[f"{pre}.bn.running_mean"],
                                      P[f"{pre}.bn.running_var"], eps)
        y = oracle.affine_act(y, scale, shift, io.act)
    return y + res if res is not None else y


def normwise(got, ref):
    got = np.asarray(got, np.float64); ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


TOL = 2e-2   # the north_star's bf16 relative tolerance


def argmax_last(scores_flat, nc, a_s):
    """Per-anchor class argmax (last maximal class wins, Rust max_by), the
    best logit and the top-2 margin."""
    out, best, margins, base = [], [], [], 0
    for a in a_s:
        blk = scores_flat[:, nc * base: nc * (base + a)].reshape(-1, nc, a)
        out.append(nc - 1 - np.argmax(blk[:, ::-1, :], axis=1))
        srt = np.sort(blk, axis=1)
        best.append(srt[:, -1, :])
        margins.append(srt[:, -1, :] - srt[:, -2, :])
        base += a
    return np.concatenate(out, 1), np.concatenate(best, 1), np.concatenate(margins, 1)


def detection_checks(boxes, scores, rb, rs, size, tol=TOL):
    """Detections against reference outputs rb, rs (float32 oracle): class
    argmax at every anchor whose reference top-2 logit margin exceeds
    2 * tol * std(reference logits), and the device post-process's top-k
    anchors at every rank whose reference best-class logit is separated from
    both neighbours' by that margin.  Returns (checked anchors, argmax
    mismatches, checked ranks, top-k mismatches, detection counts)."""
    import torch
    a_s = [(size // s) ** 2 for s in (8, 16, 32)]
    margin_min = 2.0 * tol * float(np.std(np.asarray(rs, np.float64)))
    cg, _, _ = argmax_last(scores, 80, a_s)
    cr, best, margin = argmax_last(rs, 80, a_s)
    sure = margin > margin_min
    mism = int(np.sum(cg[sure] != cr[sure]))
    got = ctx().detect_postprocess(dev(boxes), dev(scores), 80, size, size, (8, 16, 32), 0.25, 300)
    torch.cuda.synchronize()
    gc, _, _, gan, _ = [t.cpu().numpy() for t in got]
    rc, _, _, ran, _ = oracle.detect_postprocess(rb, rs, 80, size, size, (8, 16, 32), 0.25, 300)
    topk_bad, topk_n = 0, 0
    for b in range(boxes.shape[0]):
        k = int(min(gc[b], rc[b]))
        lg = best[b][ran[b, :k]]   # reference best-class logit of each ranked anchor
        sep = np.ones(k, bool)
        gap = (lg[:-1] - lg[1:]) > margin_min
        sep[1:] &= gap
        sep[:-1] &= gap
        topk_bad += int(np.sum(gan[b, :k][sep] != ran[b, :k][sep]))
        topk_n += int(np.sum(sep))
    return int(sure.sum()), mism, topk_n, topk_bad, (list(gc), list(rc))


def e2e_report(tag, boxes, scores, rb, rs, size):
    """Normwise errors and the detection checks against reference outputs."""
    eb, es = normwise(boxes, rb), normwise(scores, rs)
    n_am, mism, n_tk, topk_bad, counts = detection_checks(boxes, scores, rb, rs, size)
    print(f"{tag}: normwise boxes {eb:.3e} scores {es:.3e}; argmax mismatches {mism} of {n_am} anchors with "
          f"margin > 2*{TOL}*std; top-k anchor mismatches {topk_bad} of {n_tk} separated ranks; "
          f"detections {counts[0]} vs {counts[1]}")
    return eb, es, mism, topk_bad, n_am


@pytest.mark.parametrize("dtype", [vrs.BF16, vrs.FP8], ids=["bf16", "fp8"])
def test_yolo26m_bs64_640_layer_by_layer(dtype):
    import torch
    B, S = 64, 640
    desc = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="m", one2one=True)
    m = vrs.Model(ctx(), desc, B, S, S, dtype, 1e-3, autotune=2 if dtype == vrs.FP8 else 1)
    # the committed tile plan: every kernel the bench line runs is the one checked here
    import bench
    plan = bench.load_plan(bench.plan_path("m", "fp8_forced" if dtype == vrs.FP8 else "bf16", B, S),
                           [pre for pre, _, _ in m.conv_info()])
    assert plan is not None, "committed plan missing or out of step with the model's convs"
    m.set_plan(plan)
    P32 = seeded_params(m.params(), 0)
    P = {k: (bf16_round(v) if v.ndim == 4 else v) for k, v in P32.items()}
    x32 = np.random.default_rng(7).uniform(0, 1, (B, 3, S, S)).astype(np.float32)
    x = bf16_round(x32)
    m.load(P)
    xd = dev(x)
    if dtype == vrs.FP8:
        m.calibrate(xd)
    outs = m.forward(xd)
    torch.cuda.synchronize()
    info = m.conv_info()
    ios = []
    for i, (pre, f8, sc) in enumerate(info):
        io = m.conv_io(i)
        io.prefix = pre
        io.index = i
        ios.append(io)
    if dtype == vrs.FP8:
        n_f8 = sum(io.fp8 for io in ios)
        eligible = sum(1 for io in ios if io.groups == 1 and not io.stem and io.cin % 64 == 0 and
                       (io.up.data is None or io.up.c % 64 == 0))
        print(f"fp8 forced: {n_f8} of {len(ios)} convs on e4m3 ({eligible} eligible)")
        assert n_f8 == eligible and n_f8 > 60
    by_launch = {io.launch: io for io in ios if io.launch >= 0}
    n = len(m.launch_names())
    worst = []
    n_e4m3 = 0
    for li in range(n):
        io = by_launch.get(li)
        if io is not None:
            if io.stem == 2:   # stem pair: the input is the stem of the image, computed on chip
                xin = bf16_round(conv_reference(ios[io.index - 1], P, 1e-3, x[list(IMAGES)], None))
            elif io.fused_in:   # a fused pair: the input is the conv before it, computed on chip
                prev = ios[io.index - 1]
                xprev = read_view(prev.x, prev.dtype, IMAGES, prev.x_e4m3, prev.x_step)
                xin = bf16_round(conv_reference(prev, P, 1e-3, xprev, None))
            elif io.stem:
                xin = x[list(IMAGES)]
            else:
                xin = read_view(io.x, io.dtype, IMAGES, io.x_e4m3, io.x_step)
                if io.up.data is not None:   # fused upsample: the first up.c channels are up2x(source)
                    src = read_view(io.up, io.dtype, IMAGES, io.up_e4m3, io.up_step)
                    xin[:, :io.up.c] = oracle.upsample_nearest(src)
            res = read_view(io.res, io.dtype, IMAGES, io.res_e4m3, io.res_step) if io.res.data is not None else None
        m.run_launches(li, 1)
        torch.cuda.synchronize()
        if io is None:
            continue
        ho = (xin.shape[2] + 2 * (io.k // 2) - io.k) // io.stride + 1
        wo = (xin.shape[3] + 2 * (io.k // 2) - io.k) // io.stride + 1
        got = (read_view(io.y, io.dtype, IMAGES, io.y_e4m3, io.y_step) if io.y.data is not None
               else read_flat(io, outs, IMAGES, ho, wo))
        ref = conv_reference(io, P, 1e-3, xin, res)
        if io.y_e4m3:
            # stored as e4m3: the e4m3 rounding of a value within the bar
            lo, hi = e4m3_bracket(ref, io.y_step)
            bad = int(np.sum((got < lo) | (got > hi)))
            assert bad == 0, (io.prefix, "fp8 e4m3 output", bad)
            n_e4m3 += 1
            continue
        err = rel_err(got, ref, 1e-1)
        worst.append((err, io.prefix, bool(io.fp8)))
        assert err < 2e-2, (io.prefix, "fp8" if io.fp8 else "bf16", err)
    worst.sort(reverse=True)
    print(f"{len(worst) + n_e4m3} convs checked on their own device inputs ({n_e4m3} with e4m3 outputs, held to "
          f"the e4m3 bracket of the bar); largest errors of the others: " +
          ", ".join(f"{p}{' (fp8)' if f else ''} {e:.2e}" for e, p, f in worst[:5]))
    if dtype == vrs.FP8:
        n_x8 = sum(io.x_e4m3 for io in ios)
        print(f"fp8: {n_x8} convs read e4m3 inputs, {n_e4m3} write e4m3 outputs")

    # end to end against the plain float32 oracle (and the precision-matched one)
    boxes, scores = [o.cpu().numpy() for o in outs]
    assert np.all(np.isfinite(boxes)) and np.all(np.isfinite(scores))
    tag = "fp8" if dtype == vrs.FP8 else "bf16"
    for i in IMAGES:
        rb32, rs32 = Y.yolo26(80, "m")(Y.Params(P32, eps=1e-3), x32[i:i + 1])
        eb, es, mism, topk_bad, n_am = e2e_report(f"yolo26m {tag} bs64 image {i} vs float32", boxes[i:i + 1],
                                                  scores[i:i + 1], rb32, rs32, S)
        fp8 = {io.prefix: io.in_scale for io in ios if io.fp8}
        store8 = {io.prefix: io.y_step for io in ios if io.y_e4m3}
        rbq, rsq = Y.yolo26(80, "m")(Y.Params(P, eps=1e-3, act_q=bf16_round, fp8=fp8, store8=store8),
                                     x[i:i + 1])
        qb, qs, _, _, _ = e2e_report(f"yolo26m {tag} bs64 image {i} vs the same-precision emulation",
                                     boxes[i:i + 1], scores[i:i + 1], rbq, rsq, S)
        if dtype == vrs.BF16:
            assert eb < 2e-2 and es < 2e-2, (eb, es)
            # the detection contract: most anchors clear the margin, none flips
            assert n_am > 0.5 * 8400 and mism == 0, (n_am, mism)
            assert topk_bad == 0, topk_bad
        else:
            # the stated fp8 bar (module docstring): against float32 and against
            # the precision-matched emulation, and as accurate as the emulation
            eqb, eqs = normwise(rbq, rb32), normwise(rsq, rs32)
            print(f"fp8 emulation vs float32: boxes {eqb:.3e} scores {eqs:.3e}")
            assert eb < 0.15 and es < 0.15, (eb, es)
            assert qb < 0.13 and qs < 0.13, (qb, qs)
            assert eb < 1.2 * eqb + 5e-3 and es < 1.2 * eqs + 5e-3, (eb, eqb, es, eqs)
