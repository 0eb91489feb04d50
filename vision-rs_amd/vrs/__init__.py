"""Python binding of the vision-rs MI355X hot path (include/vrs.h) over ctypes.

The product is the C ABI in vision-rs_amd/lib/libvrs.so plus the gfx950 code
objects next to it; this module only marshals arguments.  torch provides
device memory and the current stream (plumbing); every computation runs in the
HIP kernels.  There is no CPU fallback: if the library or code objects are
missing, loading fails with an error.

Layer/op names mirror the reference crate: conv / conv_bn / dwconv /
conv_plain (blocks/conv.rs), c3k2, c3k2_psa (blocks/c3k2.rs), c2psa and
psa_attention (blocks/c2psa.rs), sppf (blocks/sppf.rs), detect
(blocks/detect.rs), yolo26 (yolo26/mod.rs).
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG, "lib")
# VRS_SO selects another build of the host library (the CPU sanitizer build of
# `make -C oracle sanitize`); the code objects always come from LIB_DIR
SO = os.environ.get("VRS_SO") or os.path.join(LIB_DIR, "libvrs.so")

VRS_OK = 0
F32, BF16, FP8 = 0, 1, 2
ACT_NONE, ACT_SILU = 0, 1
BLOCK_CONV, BLOCK_C3K2, BLOCK_C3K2_PSA, BLOCK_C2PSA, BLOCK_SPPF, BLOCK_PSA_ATTN, BLOCK_DETECT_BOX, BLOCK_YOLO26 = \
    1, 2, 3, 4, 5, 6, 7, 8
BLOCK_DETECT = 9   # the whole Detect head on three feature maps (ch = their channels)
CONV_BN_SILU, CONV_BN, CONV_PLAIN = 0, 1, 2
TILE_AUTO, TILE_128x128, TILE_256x128, TILE_128x256, TILE_64x256, TILE_32x256, TILE_256x256, TILE_K32 = (
    0, 1, 2, 3, 4, 5, 6, 0x100)
TILE_PERSIST = 0x200
TILE_K128 = 0x400   # fp8: 128-deep K steps (256x256 with e4m3 input, Cin % 128 == 0)
TILE_H3 = 7   # halo-tiled 3x3 stride-1 kernel (bf16)
TILE_W1_256 = 8   # weight-stationary 1x1 kernels (bf16): 256- or 128-channel weight slice in LDS
TILE_W1_128 = 9
TILE_64x64 = 10   # bf16: small maps (four times the workgroups of 128x128)
TILE_STEM_PAIR = 11   # model plans: the conv after a 64-channel stem, fused with it (bf16)
TILE_BPAIR = 12   # model plans: a bottleneck's second 3x3 conv, fused with the first (bf16)
TILE_PWPAIR = 13   # model plans: a Detect class output conv fused with the 1x1 conv before it (bf16)

ERRORS = {-1: "EINVAL", -2: "EBADSHAPE", -3: "EUNSUPPORTED", -4: "ENOMODULE", -5: "EHIP", -6: "ENOTFOUND",
          -7: "ESTATE"}


class VrsError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"vrs error {code} ({ERRORS.get(code, '?')}): {msg}")
        self.code = code


class Nhwc(C.Structure):
    _fields_ = [("data", C.c_void_p), ("n", C.c_int32), ("h", C.c_int32), ("w", C.c_int32), ("c", C.c_int32),
                ("pitch", C.c_int32), ("c_off", C.c_int32)]


class ConvDesc(C.Structure):
    _fields_ = [("k", C.c_int32), ("stride", C.c_int32), ("groups", C.c_int32), ("act", C.c_int32),
                ("dtype", C.c_int32), ("tile", C.c_int32), ("in_scale", C.c_float),
                ("x_e4m3", C.c_int32), ("y_e4m3", C.c_int32), ("res_e4m3", C.c_int32),
                ("out_step", C.c_float), ("res_step", C.c_float)]


class PsaDesc(C.Structure):
    _fields_ = [("heads", C.c_int32), ("key_dim", C.c_int32), ("head_dim", C.c_int32), ("dtype", C.c_int32)]


class DetectDesc(C.Structure):
    _fields_ = [("n", C.c_int32), ("nc", C.c_int32), ("img_h", C.c_int32), ("img_w", C.c_int32),
                ("nscales", C.c_int32), ("strides", C.c_int32 * 4), ("thr", C.c_float), ("max_det", C.c_int32)]


class MsdaDesc(C.Structure):
    _fields_ = [("n", C.c_int32), ("q", C.c_int32), ("heads", C.c_int32), ("head_dim", C.c_int32),
                ("levels", C.c_int32), ("points", C.c_int32), ("level_h", C.c_int32 * 8),
                ("level_w", C.c_int32 * 8)]


class BlockDesc(C.Structure):
    _fields_ = [("kind", C.c_int32), ("c_in", C.c_int32), ("c_out", C.c_int32), ("k", C.c_int32), ("s", C.c_int32),
                ("g", C.c_int32), ("conv_kind", C.c_int32), ("n", C.c_int32), ("c3k", C.c_int32),
                ("shortcut", C.c_int32), ("e", C.c_float), ("heads", C.c_int32), ("nc", C.c_int32),
                ("variant", C.c_int32), ("one2one", C.c_int32), ("ch", C.c_int32 * 3)]


class ConvIo(C.Structure):
    _fields_ = [("launch", C.c_int32), ("k", C.c_int32), ("stride", C.c_int32), ("groups", C.c_int32),
                ("act", C.c_int32), ("plain", C.c_int32), ("stem", C.c_int32), ("fp8", C.c_int32),
                ("in_scale", C.c_float), ("dtype", C.c_int32), ("cin", C.c_int32), ("cout", C.c_int32),
                ("x", Nhwc), ("y", Nhwc), ("res", Nhwc), ("up", Nhwc), ("out_idx", C.c_int32),
                ("out_off", C.c_int64), ("out_sb", C.c_int64), ("out_sp", C.c_int64), ("out_sc", C.c_int64),
                ("x_e4m3", C.c_int32), ("y_e4m3", C.c_int32), ("res_e4m3", C.c_int32), ("up_e4m3", C.c_int32),
                ("x_step", C.c_float), ("y_step", C.c_float), ("res_step", C.c_float), ("up_step", C.c_float),
                ("fused_in", C.c_int32)]


PLAN_FP8 = 0x10000

# Every exported symbol of include/vrs.h with its ctypes signature.
_vp, _i32, _i64, _f32, _sz = C.c_void_p, C.c_int32, C.c_int64, C.c_float, C.c_size_t
_P = C.POINTER
SIGNATURES = {
    "vrs_last_error": (C.c_char_p, []),
    "vrs_version": (C.c_char_p, []),
    "vrs_ctx_create": (C.c_int, [C.c_int, C.c_char_p, _P(_vp)]),
    "vrs_ctx_destroy": (C.c_int, [_vp]),
    "vrs_conv2d": (C.c_int, [_vp, _P(ConvDesc), _P(Nhwc), _vp, _vp, _vp, _P(Nhwc), _P(Nhwc), _vp]),
    "vrs_pack_conv_weight": (_i64, [_vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "vrs_pack_conv_weight_fp8": (_i64, [_vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "vrs_pack_stem_weight": (_i64, [_vp, _i32, _i32, _vp]),
    "vrs_conv_stem": (C.c_int, [_vp, _P(ConvDesc), _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _P(Nhwc), _vp]),
    "vrs_conv_stem_pair": (C.c_int, [_vp, _P(ConvDesc), _P(ConvDesc), _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp,
                                     _vp, _vp, _vp, _P(Nhwc), _vp]),
    "vrs_conv_bottleneck_pair": (C.c_int, [_vp, _P(ConvDesc), _P(ConvDesc), _P(Nhwc), _vp, _vp, _vp, _i32, _vp, _vp,
                                           _vp, _P(Nhwc), _P(Nhwc), _vp]),
    "vrs_conv_pointwise_pair": (C.c_int, [_vp, _P(ConvDesc), _P(ConvDesc), _P(Nhwc), _vp, _vp, _vp, _i32, _vp, _vp,
                                          _vp, _i32, _vp, C.c_int64, C.c_int64, C.c_int64, _vp]),
    "vrs_bn_fold": (C.c_int, [_vp, _vp, _vp, _vp, _f32, _i32, _vp, _vp]),
    "vrs_pack_input": (C.c_int, [_vp, _vp, _i32, _i32, _i32, _i32, _P(Nhwc), _i32, _vp]),
    "vrs_unpack_output": (C.c_int, [_vp, _P(Nhwc), _i32, _vp, _vp]),
    "vrs_sppf_pool": (C.c_int, [_vp, _P(Nhwc), _i32, _vp]),
    "vrs_upsample2x": (C.c_int, [_vp, _P(Nhwc), _P(Nhwc), _i32, _vp]),
    "vrs_psa_attention": (C.c_int, [_vp, _P(PsaDesc), _P(Nhwc), _vp, _vp, _vp, _P(Nhwc), _vp]),
    "vrs_detect_workspace_size": (_sz, [_P(DetectDesc)]),
    "vrs_detect_postprocess": (C.c_int, [_vp, _P(DetectDesc), _vp, _vp, _vp, _sz, _vp, _vp, _vp, _vp, _vp, _vp]),
    "vrs_detect_postprocess_noalloc": (C.c_int, [_vp, _P(DetectDesc), _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "vrs_detect_decode_grid": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "vrs_detect_unletterbox": (C.c_int, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "vrs_letterbox": (C.c_int, [_vp, _i32, _i32, _vp, _i64, _P(_i64), _P(_i32), _vp, _vp]),
    "vrs_msda": (C.c_int, [_vp, _P(MsdaDesc), _vp, _vp, _vp, _vp, _vp, _vp]),
    "vrs_model_create": (C.c_int, [_vp, _P(BlockDesc), _i32, _i32, _i32, _i32, _f32, _P(_vp)]),
    "vrs_model_set_autotune": (C.c_int, [_vp, _i32]),
    "vrs_model_num_params": (C.c_int, [_vp]),
    "vrs_model_param_info": (C.c_int, [_vp, _i32, _P(C.c_char_p), _P(_i32), _P(_i32)]),
    "vrs_model_load_param": (C.c_int, [_vp, C.c_char_p, _vp, _i64]),
    "vrs_model_load_safetensors": (C.c_int, [_vp, C.c_char_p, _P(_i32), _P(_i32)]),
    "vrs_model_finalize": (C.c_int, [_vp]),
    "vrs_model_num_outputs": (C.c_int, [_vp]),
    "vrs_model_output_info": (C.c_int, [_vp, _i32, _P(_i64), _P(_i32), _P(_i32)]),
    "vrs_model_forward": (C.c_int, [_vp, _vp, _P(_vp), _vp]),
    "vrs_model_capture": (C.c_int, [_vp, _vp, _P(_vp), _vp]),
    "vrs_model_replay": (C.c_int, [_vp, _vp]),
    "vrs_model_set_streams": (C.c_int, [_vp, _i32]),
    "vrs_model_num_capture_streams": (C.c_int, [_vp]),
    "vrs_model_num_launches": (C.c_int, [_vp]),
    "vrs_model_launch_name": (C.c_char_p, [_vp, _i32]),
    "vrs_model_launch_work": (C.c_int, [_vp, _i32, _P(C.c_double), _P(C.c_double)]),
    "vrs_model_run_launches": (C.c_int, [_vp, _i32, _i32, _vp]),
    "vrs_model_calibrate": (C.c_int, [_vp, _vp, _vp]),
    "vrs_model_num_convs": (C.c_int, [_vp]),
    "vrs_model_conv_info": (C.c_int, [_vp, _i32, _P(C.c_char_p), _P(_i32), _P(_f32)]),
    "vrs_model_set_plan": (C.c_int, [_vp, _P(_i32), _i32]),
    "vrs_model_get_plan": (C.c_int, [_vp, _P(_i32), _i32]),
    "vrs_model_conv_io": (C.c_int, [_vp, _i32, _P(ConvIo)]),
    "vrs_model_destroy": (C.c_int, [_vp]),
}

_lib = None


def lib():
    """Load libvrs.so (raises if it was not built: there is no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(SO):
            raise RuntimeError(f"{SO} not built: run `python vision-rs_amd/build.py` (no CPU fallback exists)")
        L = C.CDLL(SO)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> int:
    if rc < 0:
        raise VrsError(rc, lib().vrs_last_error().decode(errors="replace"))
    return rc


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(stream=None):
    if stream is not None:
        return C.c_void_p(stream)
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


class _alloc_on:
    """Allocate temporaries and outputs on the stream the kernels run on.

    torch's caching allocator ties a block to the stream current at
    allocation time; a buffer a kernel on another stream still uses could be
    handed out again once its tensor is dropped.  With an explicit stream,
    the tensors are allocated while that stream is current."""

    def __init__(self, stream, device=None):
        self.stream, self.device, self.ctx = stream, device, None

    def __enter__(self):
        if self.stream is not None:
            import torch
            self.ctx = torch.cuda.stream(torch.cuda.ExternalStream(self.stream, device=self.device))
            self.ctx.__enter__()
        return self

    def __exit__(self, *exc):
        if self.ctx is not None:
            self.ctx.__exit__(*exc)
        return False


def nhwc(t, c=None, c_off=0):
    """View of a [n, h, w, pitch] torch tensor (channels [c_off, c_off+c))."""
    n, h, w, pitch = t.shape
    return Nhwc(t.data_ptr(), n, h, w, pitch - c_off if c is None else c, pitch, c_off)


def dtype_code(torch_dtype) -> int:
    import torch
    if torch_dtype == torch.bfloat16:
        return BF16
    if torch_dtype == torch.float32:
        return F32
    raise ValueError(f"unsupported dtype {torch_dtype}")


class Context:
    """vrs_ctx: one device, all code objects loaded (CudaGraphCompiler::load analogue)."""

    def __init__(self, device: int = 0, hsaco_dir: str | None = None):
        self.handle = C.c_void_p()
        d = LIB_DIR if hsaco_dir is None else hsaco_dir
        check(lib().vrs_ctx_create(device, d.encode(), C.byref(self.handle)))
        self.device = device

    def close(self):
        if self.handle:
            lib().vrs_ctx_destroy(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- single ops --------------------------------------------------------
    def conv2d(self, x, w, scale, shift, y, k, stride=1, groups=1, act=ACT_SILU, res=None, dtype=BF16,
               stream=None, tile=TILE_AUTO, in_scale=1.0, x_e4m3=False, y_e4m3=False, out_step=0.0,
               res_e4m3=False, res_step=0.0):
        """x, y, res: Nhwc views; w/scale/shift: device tensors.  FP8: w from
        pack_conv_weight_fp8, scale including weight scale * in_scale; views of
        uint8 tensors hold e4m3 activations when x_e4m3 / y_e4m3 / res_e4m3."""
        d = ConvDesc(k, stride, groups, act, dtype, tile, in_scale, int(x_e4m3), int(y_e4m3), int(res_e4m3),
                     out_step, res_step)
        check(lib().vrs_conv2d(self.handle, C.byref(d), C.byref(x), _ptr(w), _ptr(scale), _ptr(shift),
                               C.byref(res) if res is not None else None, C.byref(y), _stream(stream)))

    def conv_stem(self, x_nchw, w, scale, shift, y, act=ACT_SILU, dtype=BF16, stream=None):
        """model.0 (3x3 s2, 3 channels) from the NCHW float32 image into NHWC view y."""
        n, c, h, w_ = x_nchw.shape
        d = ConvDesc(3, 2, 1, act, dtype, TILE_AUTO, 1.0, 0, 0, 0, 0.0, 0.0)
        check(lib().vrs_conv_stem(self.handle, C.byref(d), _ptr(x_nchw), n, c, h, w_, _ptr(w), _ptr(scale),
                                  _ptr(shift), C.byref(y), _stream(stream)))

    def conv_stem_pair(self, x_nchw, w0, scale0, shift0, w1, scale1, shift1, y, act=ACT_SILU, dtype=BF16,
                       stream=None):
        """model.0 + model.1 (3 -> 64 -> 128 channels, both 3x3 s2) in one kernel from the NCHW
        float32 image into the 128-channel NHWC view y; w0 from pack_stem_weight, w1 from
        pack_conv_weight."""
        n, c, h, w_ = x_nchw.shape
        d0 = ConvDesc(3, 2, 1, act, dtype, TILE_AUTO, 1.0, 0, 0, 0, 0.0, 0.0)
        d1 = ConvDesc(3, 2, 1, act, dtype, TILE_AUTO, 1.0, 0, 0, 0, 0.0, 0.0)
        check(lib().vrs_conv_stem_pair(self.handle, C.byref(d0), C.byref(d1), _ptr(x_nchw), n, c, h, w_, _ptr(w0),
                                       _ptr(scale0), _ptr(shift0), _ptr(w1), _ptr(scale1), _ptr(shift1),
                                       C.byref(y), _stream(stream)))

    def conv_bottleneck_pair(self, x, w1, scale1, shift1, c_hidden, w2, scale2, shift2, y, res=None, dtype=BF16,
                             stream=None):
        """A bottleneck's 3x3 -> 3x3 (+ residual res) in one kernel: x, y, res Nhwc
        views; w1 / w2 from pack_conv_weight ([c_hidden][3][3][c], [c][3][3][c_hidden])."""
        d1 = ConvDesc(3, 1, 1, ACT_SILU, dtype, TILE_AUTO, 1.0, 0, 0, 0, 0.0, 0.0)
        d2 = ConvDesc(3, 1, 1, ACT_SILU, dtype, TILE_AUTO, 1.0, 0, 0, 0, 0.0, 0.0)
        check(lib().vrs_conv_bottleneck_pair(self.handle, C.byref(d1), C.byref(d2), C.byref(x), _ptr(w1),
                                             _ptr(scale1), _ptr(shift1), c_hidden, _ptr(w2), _ptr(scale2),
                                             _ptr(shift2), C.byref(res) if res is not None else None, C.byref(y),
                                             _stream(stream)))

    def conv_pointwise_pair(self, x, w1, scale1, shift1, c_mid, w2, scale2, shift2, nc, y, sb, sp, sc, stream=None):
        """A Detect class branch's last 1x1 conv (BN + SiLU) and its 1x1 conv_plain in one kernel:
        x an Nhwc view; w1 / w2 from pack_conv_weight ([c_mid][c], [nc][c_mid]); y a float32 device
        tensor written at y[b*sb + p*sp + co*sc]."""
        d1 = ConvDesc(1, 1, 1, ACT_SILU, BF16, TILE_AUTO, 1.0, 0, 0, 0, 0.0, 0.0)
        d2 = ConvDesc(1, 1, 1, ACT_NONE, BF16, TILE_AUTO, 1.0, 0, 0, 0, 0.0, 0.0)
        check(lib().vrs_conv_pointwise_pair(self.handle, C.byref(d1), C.byref(d2), C.byref(x), _ptr(w1),
                                            _ptr(scale1), _ptr(shift1), c_mid, _ptr(w2), _ptr(scale2),
                                            _ptr(shift2), nc, _ptr(y), sb, sp, sc, _stream(stream)))

    def pack_input(self, x_nchw, y, dtype, stream=None):
        n, c, h, w = x_nchw.shape
        check(lib().vrs_pack_input(self.handle, _ptr(x_nchw), n, c, h, w, C.byref(y), dtype, _stream(stream)))

    def unpack_output(self, x, dtype, y_nchw, stream=None):
        check(lib().vrs_unpack_output(self.handle, C.byref(x), dtype, _ptr(y_nchw), _stream(stream)))

    def sppf_pool(self, buf, dtype, stream=None):
        check(lib().vrs_sppf_pool(self.handle, C.byref(buf), dtype, _stream(stream)))

    def upsample2x(self, x, y, dtype, stream=None):
        check(lib().vrs_upsample2x(self.handle, C.byref(x), C.byref(y), dtype, _stream(stream)))

    def psa_attention(self, qkv, pe_w, pe_scale, pe_shift, out, heads, dtype, stream=None):
        d = PsaDesc(heads, 32, 64, dtype)
        check(lib().vrs_psa_attention(self.handle, C.byref(d), C.byref(qkv), _ptr(pe_w), _ptr(pe_scale),
                                      _ptr(pe_shift), C.byref(out), _stream(stream)))

    def detect_postprocess(self, boxes, scores, nc, img_h, img_w, strides=(8, 16, 32), thr=0.25, max_det=300,
                           stream=None, outs=None, workspace=None):
        """outs: the (count, score, cls, anchor, xywh) of an earlier call with
        the same shapes, written again instead of allocated; workspace: a
        uint8 device tensor of at least vrs_detect_workspace_size bytes."""
        import torch
        n = boxes.shape[0]
        st = (C.c_int32 * 4)(*list(strides), *([0] * (4 - len(strides))))
        d = DetectDesc(n, nc, img_h, img_w, len(strides), st, thr, max_det)
        ws_bytes = lib().vrs_detect_workspace_size(C.byref(d))
        if ws_bytes == 0:
            raise VrsError(-1, lib().vrs_last_error().decode(errors="replace"))
        dev = boxes.device
        with _alloc_on(stream, dev):   # the workspace is dropped on return: allocate it on the launch stream
            if workspace is not None:
                ws = workspace
                if ws.numel() * ws.element_size() < ws_bytes:
                    raise VrsError(-1, f"detect_postprocess: workspace of {ws.numel()} bytes, {ws_bytes} needed")
            else:
                ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
            if outs is not None:
                count, score, cls, anchor, xywh = outs
            else:
                count = torch.empty(n, dtype=torch.int32, device=dev)
                score = torch.empty(n, max_det, dtype=torch.float32, device=dev)
                cls = torch.empty(n, max_det, dtype=torch.int32, device=dev)
                anchor = torch.empty(n, max_det, dtype=torch.int32, device=dev)
                xywh = torch.empty(n, max_det, 4, dtype=torch.float32, device=dev)
            check(lib().vrs_detect_postprocess(self.handle, C.byref(d), _ptr(boxes), _ptr(scores), _ptr(ws),
                                               ws_bytes, _ptr(count), _ptr(score), _ptr(cls), _ptr(anchor),
                                               _ptr(xywh), _stream(stream)))
        if outs is not None:
            return outs
        return count, score, cls, anchor, xywh

    def detect_postprocess_noalloc(self, boxes, scores, nc, img_h, img_w, outs, strides=(8, 16, 32), thr=0.25,
                                   stream=None):
        """vrs_detect_postprocess_noalloc: the same post-process with the
        library's fixed device workspace (nothing allocated); outs = the
        caller's (count, score, cls, anchor, xywh) tensors, max_det from
        their shape."""
        count, score, cls, anchor, xywh = outs
        n, max_det = score.shape
        st = (C.c_int32 * 4)(*list(strides), *([0] * (4 - len(strides))))
        d = DetectDesc(n, nc, img_h, img_w, len(strides), st, thr, max_det)
        check(lib().vrs_detect_postprocess_noalloc(self.handle, C.byref(d), _ptr(boxes), _ptr(scores), _ptr(count),
                                                   _ptr(score), _ptr(cls), _ptr(anchor), _ptr(xywh),
                                                   _stream(stream)))
        return outs

    def detect_unletterbox(self, count, xywh, orig_wh, img_size, stream=None):
        """Letterbox-pixel xywh [n][max_det][4] (detect_postprocess) -> boxes
        normalised to each original image; orig_wh [n][2] int32 on the device."""
        import torch
        n, max_det, _ = xywh.shape
        with _alloc_on(stream, xywh.device):
            out = torch.empty_like(xywh)
        check(lib().vrs_detect_unletterbox(self.handle, n, max_det, img_size, _ptr(orig_wh), _ptr(count),
                                           _ptr(xywh), _ptr(out), _stream(stream)))
        return out

    def letterbox(self, rgb, offsets, wh, img_size, out=None, stream=None):
        """Letterbox n RGB8 images held in one flat uint8 device tensor (image
        i: wh[i] = (w, h) pixels at byte offsets[i]) into the model input
        [n][3][img_size][img_size] float32 (preprocess_image_raw)."""
        import torch
        n = len(wh)
        if out is None:
            with _alloc_on(stream, rgb.device):
                out = torch.empty(n, 3, img_size, img_size, dtype=torch.float32, device=rgb.device)
        offs = (C.c_int64 * n)(*[int(o) for o in offsets])
        dims = (C.c_int32 * (2 * n))(*[int(v) for w_h in wh for v in w_h])
        check(lib().vrs_letterbox(self.handle, n, img_size, _ptr(rgb), rgb.numel() * rgb.element_size(), offs, dims,
                                  _ptr(out), _stream(stream)))
        return out

    def detect_decode_grid(self, boxes, ax, ay, strides, out, stream=None):
        n, _, a = boxes.shape
        check(lib().vrs_detect_decode_grid(self.handle, _ptr(boxes), _ptr(ax), _ptr(ay), _ptr(strides), n, a,
                                           _ptr(out), _stream(stream)))

    def msda(self, value, shapes, ref, off, attw, out, stream=None):
        n, s, heads, dh = value.shape
        _, q, _, L, P, _ = off.shape
        lh = (C.c_int32 * 8)(*[h for h, _ in shapes], *([0] * (8 - L)))
        lw = (C.c_int32 * 8)(*[w for _, w in shapes], *([0] * (8 - L)))
        d = MsdaDesc(n, q, heads, dh, L, P, lh, lw)
        check(lib().vrs_msda(self.handle, C.byref(d), _ptr(value), _ptr(ref), _ptr(off), _ptr(attw), _ptr(out),
                             _stream(stream)))


def pack_conv_weight(w_oihw, groups=1, cin_pad=None, dtype=BF16):
    """Host repack (numpy float32 OIHW) -> bytes in the device layout
    (dense [Cout][k][k][cin_pad]; depthwise tap-major [k*k][C]), dtype elements."""
    import numpy as np
    w = np.ascontiguousarray(w_oihw, dtype=np.float32)
    cout, cin_g, k, _ = w.shape
    cin_pad = cin_g if cin_pad is None else cin_pad
    n = check(lib().vrs_pack_conv_weight(None, cout, cin_g, k, groups, cin_pad, dtype, None))
    out = np.empty(n, np.uint8)
    check(lib().vrs_pack_conv_weight(w.ctypes.data, cout, cin_g, k, groups, cin_pad, dtype, out.ctypes.data))
    return out


def pack_stem_weight(w_oihw, dtype=BF16):
    """Host pack of the stem weights [Cout][3][3][3] -> [ceil32(Cout)][32] (k = c*9 + ky*3 + kx)."""
    import numpy as np
    w = np.ascontiguousarray(w_oihw, dtype=np.float32)
    n = check(lib().vrs_pack_stem_weight(None, w.shape[0], dtype, None))
    out = np.empty(n, np.uint8)
    check(lib().vrs_pack_stem_weight(w.ctypes.data, w.shape[0], dtype, out.ctypes.data))
    return out


def pack_conv_weight_fp8(w_oihw, cin_pad=None):
    """Host e4m3 pack (dense only): (bytes [Cout][k][k][cin_pad], per-channel
    weight scales absmax/448)."""
    import numpy as np
    w = np.ascontiguousarray(w_oihw, dtype=np.float32)
    cout, cin, k, _ = w.shape
    cin_pad = cin if cin_pad is None else cin_pad
    n = check(lib().vrs_pack_conv_weight_fp8(None, cout, cin, k, cin_pad, None, None))
    out = np.empty(n, np.uint8)
    sc = np.empty(cout, np.float32)
    check(lib().vrs_pack_conv_weight_fp8(w.ctypes.data, cout, cin, k, cin_pad, out.ctypes.data, sc.ctypes.data))
    return out, sc


def bn_fold(gamma, beta, mean, var, eps):
    import numpy as np
    c = gamma.shape[0]
    s = np.empty(c, np.float32); t = np.empty(c, np.float32)
    arrs = [np.ascontiguousarray(a, np.float32) for a in (gamma, beta, mean, var)]
    check(lib().vrs_bn_fold(*[a.ctypes.data for a in arrs], eps, c, s.ctypes.data, t.ctypes.data))
    return s, t


class Model:
    """vrs_model: a recorded block/network with its parameters and buffers.

    Mirrors the reference's flow: build closures -> load_param_f32 per name ->
    forward / capture_graph + run_inplace."""

    def __init__(self, ctx, desc: BlockDesc, batch: int, h: int, w: int, dtype=BF16, bn_eps=1e-3,
                 autotune=True):
        """ctx=None records the layers only (params()/output_shapes() work without a GPU).
        autotune: False/0 heuristic tiles, True/1 timed per layer, 2 (fp8
        models) timed among fp8 tiles with every eligible conv kept on fp8."""
        self.ctx = ctx
        self.desc = desc
        self.batch, self.h, self.w, self.dtype = batch, h, w, dtype
        self.handle = C.c_void_p()
        check(lib().vrs_model_create(ctx.handle if ctx is not None else None, C.byref(desc), batch, h, w, dtype,
                                     bn_eps, C.byref(self.handle)))
        check(lib().vrs_model_set_autotune(self.handle, int(autotune)))

    def params(self):
        """[(name, shape)] in recording order (the reference's name_scope paths)."""
        out = []
        n = check(lib().vrs_model_num_params(self.handle))
        for i in range(n):
            name = C.c_char_p()
            dims = (C.c_int32 * 4)()
            nd = C.c_int32()
            check(lib().vrs_model_param_info(self.handle, i, C.byref(name), dims, C.byref(nd)))
            out.append((name.value.decode(), tuple(dims[j] for j in range(nd.value))))
        return out

    def load(self, P: dict):
        import numpy as np
        for name, shape in self.params():
            a = np.ascontiguousarray(P[name], dtype=np.float32).reshape(shape)
            check(lib().vrs_model_load_param(self.handle, name.encode(), a.ctypes.data, a.size))
        check(lib().vrs_model_finalize(self.handle))
        return self

    def load_safetensors(self, path, finalize=True):
        """load_weights_from_safetensors: parameters by name from a local file;
        returns (loaded, missing) counts.  finalize=True folds BN and uploads
        (every parameter must then have been found)."""
        n_loaded, n_missing = C.c_int32(), C.c_int32()
        check(lib().vrs_model_load_safetensors(self.handle, os.fsencode(path), C.byref(n_loaded),
                                               C.byref(n_missing)))
        if finalize:
            check(lib().vrs_model_finalize(self.handle))
        return n_loaded.value, n_missing.value

    def output_shapes(self):
        out = []
        for i in range(check(lib().vrs_model_num_outputs(self.handle))):
            numel = C.c_int64()
            dims = (C.c_int32 * 4)()
            nd = C.c_int32()
            check(lib().vrs_model_output_info(self.handle, i, C.byref(numel), dims, C.byref(nd)))
            out.append(tuple(dims[j] for j in range(nd.value)))
        return out

    def alloc_outputs(self, device="cuda"):
        import torch
        return [torch.empty(s, dtype=torch.float32, device=device) for s in self.output_shapes()]

    def forward(self, x, outs=None, stream=None):
        if outs is None:
            with _alloc_on(stream, x.device):
                outs = self.alloc_outputs(x.device)
        ptrs = (C.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
        check(lib().vrs_model_forward(self.handle, _ptr(x), ptrs, _stream(stream)))
        return outs

    def capture(self, x, outs, stream):
        ptrs = (C.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
        check(lib().vrs_model_capture(self.handle, _ptr(x), ptrs, C.c_void_p(stream)))

    def replay(self, stream):
        check(lib().vrs_model_replay(self.handle, C.c_void_p(stream)))

    def set_streams(self, n):
        check(lib().vrs_model_set_streams(self.handle, n))

    def num_capture_streams(self):
        return lib().vrs_model_num_capture_streams(self.handle)

    def launch_names(self):
        n = lib().vrs_model_num_launches(self.handle)
        return [lib().vrs_model_launch_name(self.handle, i).decode() for i in range(n)]

    def launch_work(self):
        """[(flops, bytes)] per launch of the prepared forward."""
        out = []
        for i in range(lib().vrs_model_num_launches(self.handle)):
            f, b = C.c_double(), C.c_double()
            check(lib().vrs_model_launch_work(self.handle, i, C.byref(f), C.byref(b)))
            out.append((f.value, b.value))
        return out

    def calibrate(self, x, stream=None):
        """FP8 models: activation scales from one bf16 forward of x."""
        check(lib().vrs_model_calibrate(self.handle, _ptr(x), _stream(stream)))

    def conv_info(self):
        """[(prefix, runs_on_fp8, in_scale)] per conv in build order."""
        out = []
        for i in range(check(lib().vrs_model_num_convs(self.handle))):
            pre, f8, sc = C.c_char_p(), C.c_int32(), C.c_float()
            check(lib().vrs_model_conv_info(self.handle, i, C.byref(pre), C.byref(f8), C.byref(sc)))
            out.append((pre.value.decode(), bool(f8.value), sc.value))
        return out

    def set_plan(self, plan):
        """Tile plan to apply at finalize instead of autotuning (list of ints,
        one per conv; see get_plan)."""
        arr = (C.c_int32 * len(plan))(*[int(v) for v in plan])
        check(lib().vrs_model_set_plan(self.handle, arr, len(plan)))

    def get_plan(self):
        """Per-conv tile codes in use (| PLAN_FP8 for convs on e4m3)."""
        n = check(lib().vrs_model_get_plan(self.handle, None, 0))
        arr = (C.c_int32 * n)()
        check(lib().vrs_model_get_plan(self.handle, arr, n))
        return list(arr)

    def conv_io(self, i):
        """vrs_conv_io of conv i (launch index, views of its input, output,
        residual and fused-upsample source)."""
        io = ConvIo()
        check(lib().vrs_model_conv_io(self.handle, i, C.byref(io)))
        return io

    def run_launches(self, first, count, stream=None):
        check(lib().vrs_model_run_launches(self.handle, first, count, _stream(stream)))

    def close(self):
        if self.handle:
            lib().vrs_model_destroy(self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def block(kind, c_in, c_out=0, k=1, s=1, g=1, conv_kind=CONV_BN_SILU, n=1, c3k=False, shortcut=False, e=0.5,
          heads=0, nc=80, variant="m", one2one=True, ch=(0, 0, 0)):
    return BlockDesc(kind, c_in, c_out, k, s, g, conv_kind, n, int(c3k), int(shortcut), e, heads, nc,
                     ord(variant), int(one2one), (C.c_int32 * 3)(*ch))
