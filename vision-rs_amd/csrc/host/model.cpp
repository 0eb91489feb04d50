// Model runtime: the reference's layer closures (src/models/yolo/yolo26/) restated as
// destination-passing builders over planned NHWC buffers, plus the
// LoadedModel roles (parameter upload, forward, graph capture and replay).
//
// The reference records a symbolic graph (ChannelCat / ChannelChunk / Add /
// UpsampleNearest2d nodes, blocks/c3k2.rs:26-41, blocks/concat.rs:24-38) and
// lowers every node to a kernel.  Here each producer writes straight into the
// channel slice of the buffer its consumer reads, so concat and chunk are
// free, residual adds run in the producing conv's epilogue, and only convs,
// the SPPF pool, upsample and PSA attention launch kernels.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <memory>
#include <string>

#include "vrs_internal.h"

using namespace vrs;

namespace {

enum ConvKind { CK_BN_SILU = 0, CK_BN = 1, CK_PLAIN = 2 };

struct V {  // channel slice of a model buffer
  int buf = -1, c_off = 0, c = 0;
};

struct Buf {
  int h = 0, w = 0, pitch = 0;
  void* dev = nullptr;
  // VRS_FP8 models: stored as e4m3 on `step` (every reader and writer is an
  // fp8 conv); buffers read together by one conv (input + fused-upsample
  // source) share a step group
  bool f8 = false;
  int grp = -1;
  float step = 0.f;
};

struct Param {
  std::string name;
  std::vector<int32_t> dims;
  std::vector<float> host;
  bool loaded = false;
};

struct ConvStep {
  std::string pre;
  int kind = CK_BN_SILU;
  bool dw = false;
  int groups = 1;            // 1 < groups < channels: grouped conv_bn (dw: groups == channels)
  int k = 1, s = 1, cin = 0, cout = 0;
  V x, y;
  bool has_res = false;
  V res;
  // flat float32 output (detect head / block outputs): output index + layout
  int out_idx = -1;
  int64_t out_off = 0, sb = 0, sp = 0, sc = 0;
  int tile = VRS_TILE_AUTO;  // chosen at finalize (autotune) for dense NHWC convs
  bool stem = false;         // fused input conv: reads the NCHW float32 image (no x buffer)
  int cin_real = 0;          // unpadded input channels (work accounting)
  // device parameters (finalize)
  void* w = nullptr;
  float* scale = nullptr;
  float* shift = nullptr;
  // VRS_FP8 models: dense convs with Cin % 64 == 0 run on e4m3
  bool f8 = false;
  void* w8 = nullptr;               // e4m3 weights [Cout][k][k][Cin]
  float* scale8 = nullptr;          // BN scale * weight scale * in_scale (after calibration)
  std::vector<float> scale8_host;   // BN scale * weight scale
  float in_scale = 0.f;             // activation step (power of two), 0 = not calibrated
  int tile8 = VRS_TILE_AUTO;
  // autotune: false when this layer's best bf16 tile beat its best fp8 tile
  // (the layer then runs bf16 in the fp8 model)
  bool run_f8 = true;
  // fused nearest-2x upsample: input channels [0, up.c) come from this
  // half-resolution view (the upsample step feeding them was dropped)
  bool has_up = false;
  V up;
};

// A launch's memory accesses, for the dependency graph of a capture:
// resource (>= 0 an activation buffer, kResInput the input image, kResOut - i
// output i) and a channel range [c0, c1).
struct Access {
  int res, c0, c1;
};
struct LaunchIO {
  std::vector<Access> rd, wr;
};
constexpr int kResInput = -1, kResOut = -2;

struct Step {
  enum Type { PACK, CONV, POOL, UP, ATTN, UNPACK, STEM } type;
  int conv = -1;      // CONV / ATTN (the PE conv's parameters)
  V a, b;             // PACK: b = dest; POOL: a; UP: a -> b; ATTN: a = qkv, b = out; UNPACK: a
  int heads = 0;
  int out_idx = -1;   // UNPACK
  // PACK: the input tensor's channels and size, and its float offset in the
  // model input (a multi-input block's tensors lie back to back)
  int in_c = 0, in_h = 0, in_w = 0;
  int64_t in_off = 0;
  // independent chain this step belongs to (-1: the network's trunk): the
  // Detect head's six chains (box and class branch of each scale) read the
  // neck and write only their slices of the outputs, so a captured forward
  // may run them on streams of their own
  int branch = -1;
};

}  // namespace

struct vrs_model {
  vrs_ctx* ctx = nullptr;
  vrs_block_desc desc{};
  int batch = 0, in_c = 0, in_h = 0, in_w = 0, dtype = VRS_BF16;
  float eps = 1e-3f;
  std::vector<Buf> bufs;
  std::vector<Param> params;
  std::unordered_map<std::string, int> pidx;
  std::vector<ConvStep> convs;
  std::vector<Step> steps;
  std::vector<std::vector<int32_t>> out_dims;
  bool finalized = false;
  // 0: shape heuristic; 1: time every tile per layer (fp8 models: also fp8
  // against bf16); 2 (fp8 models): time only the fp8 tiles, every eligible
  // conv stays on fp8
  int autotune = 1;
  // per-conv tile plan set by the caller (replaces autotuning); empty = none
  std::vector<int32_t> plan;
  std::vector<void*> allocs;
  // prepared launches for the last (x, outputs) pointers
  std::vector<Launch> launches;
  std::vector<std::string> labels;
  std::vector<int> branch;       // per launch: its step's chain tag (-1: trunk)
  std::vector<LaunchIO> io;      // per launch: what it reads and writes
  std::vector<int> conv_launch;  // per conv: index of its kernel launch (-1: none)
  int streams = 3;               // capture concurrency: the trunk plus side streams for the Detect chains
  std::vector<hipStream_t> side; // extra capture streams (default priority)
  const float* prep_x = nullptr;
  std::vector<float*> prep_outs;
  // the captured forward: one graph; with several capture streams its
  // launches form parallel branches joined by the captured cross-stream
  // waits, which the runtime replays on parallel hardware queues
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int capture_streams = 0;       // streams the last capture used
  std::vector<hipEvent_t> cap_evs;   // the events the capture recorded and waited for
  // fp8: calibrated scales; calib_mode runs every conv on bf16 with an
  // absmax reduction in front of each fp8 conv (slot = conv index)
  bool calibrated = false;
  bool calib_mode = false;
  unsigned* absmax = nullptr;   // slots: convs, then buffers
};

namespace {

std::string J(const std::string& pre, const std::string& n) { return pre.empty() ? n : pre + "." + n; }

// element type of activations and of every non-fp8 kernel
int act_dt(const vrs_model* m) { return m->dtype == VRS_FP8 ? VRS_BF16 : m->dtype; }

// release the captured graph (a later capture rebuilds it)
void drop_graphs(vrs_model* m) {
  if (m->exec) {
    // a replay may still run; the graph and the events it was captured
    // from are released only after it
    (void)hipDeviceSynchronize();
    (void)hipGraphExecDestroy(m->exec);
  }
  if (m->graph) (void)hipGraphDestroy(m->graph);
  m->exec = nullptr;
  m->graph = nullptr;
  // the runtime's graph may refer to the capture's events: they go after it
  for (hipEvent_t e : m->cap_evs) (void)hipEventDestroy(e);
  m->cap_evs.clear();
}

class Builder {
 public:
  explicit Builder(vrs_model* m) : m_(m) {}

  V alloc(int h, int w, int c) {
    Buf b;
    b.h = h; b.w = w; b.pitch = c;
    m_->bufs.push_back(b);
    return V{(int)m_->bufs.size() - 1, 0, c};
  }
  static V slice(V v, int off, int c) { return V{v.buf, v.c_off + off, c}; }
  int H(V v) const { return m_->bufs[v.buf].h; }
  int W(V v) const { return m_->bufs[v.buf].w; }

  void add_param(const std::string& name, std::vector<int32_t> dims) {
    if (m_->pidx.count(name)) return;
    Param p;
    p.name = name;
    p.dims = std::move(dims);
    m_->pidx[name] = (int)m_->params.size();
    m_->params.push_back(std::move(p));
  }

  int conv_common(const std::string& pre, V x, int cout, int k, int s, int kind, bool dw, int groups = 1) {
    ConvStep c;
    c.pre = pre; c.kind = kind; c.dw = dw; c.groups = groups; c.k = k; c.s = s; c.cin = x.c; c.cout = cout; c.x = x;
    const int cin_g = dw ? 1 : groups > 1 ? x.c / groups : real_cin(x);
    c.cin_real = real_cin(x);
    if (kind == CK_PLAIN) {
      add_param(J(pre, "weight"), {cout, cin_g, k, k});
      add_param(J(pre, "bias"), {cout});
    } else {
      add_param(J(pre, "conv.weight"), {cout, cin_g, k, k});
      for (const char* n : {"bn.weight", "bn.bias", "bn.running_mean", "bn.running_var"}) add_param(J(pre, n), {cout});
    }
    m_->convs.push_back(c);
    return (int)m_->convs.size() - 1;
  }

  // conv() / conv_bn(): blocks/conv.rs:31-69 (optional residual = elem_add of the caller)
  void conv(const std::string& pre, V x, V y, int k, int s, int kind, const V* res = nullptr) {
    const int i = conv_common(pre, x, y.c, k, s, kind, false);
    m_->convs[i].y = y;
    if (res) { m_->convs[i].has_res = true; m_->convs[i].res = *res; }
    push_conv(i);
  }
  // dwconv() (SiLU) and conv_bn(g = c) (no act): blocks/conv.rs:53-85
  void dwconv(const std::string& pre, V x, V y, int k, int s, int kind) {
    const int i = conv_common(pre, x, y.c, k, s, kind, true);
    m_->convs[i].y = y;
    push_conv(i);
  }
  // conv_bn() with 1 < g < channels (blocks/conv.rs:51-69)
  void gconv(const std::string& pre, V x, V y, int k, int s, int kind, int g) {
    // the input view without the packed input's zero channels (they would
    // shift every group's channel range)
    const int i = conv_common(pre, slice(x, 0, real_cin(x)), y.c, k, s, kind, false, g);
    m_->convs[i].y = y;
    push_conv(i);
  }
  // conv() or conv_plain() writing float32 into a flat output (out_idx)
  void conv_flat(const std::string& pre, V x, int cout, int k, int kind, int out_idx, int64_t off, int64_t sb,
                 int64_t sp, int64_t sc) {
    const int i = conv_common(pre, x, cout, k, 1, kind, false);
    ConvStep& c = m_->convs[i];
    c.out_idx = out_idx; c.out_off = off; c.sb = sb; c.sp = sp; c.sc = sc;
    push_conv(i);
  }

  // bottleneck.rs:37-49 (c -> c/2 -> c) and :51-63 (c -> c -> c), 3x3 convs
  void bottleneck(const std::string& pre, V x, V y, int c, bool shortcut, bool inner_half) {
    const int ci = inner_half ? (int)(c * 0.5f) : c;
    V t = alloc(H(x), W(x), ci);
    conv(J(pre, "cv1"), x, t, 3, 1, CK_BN_SILU);
    conv(J(pre, "cv2"), t, y, 3, 1, CK_BN_SILU, shortcut ? &x : nullptr);
  }

  // c3k2.rs:46-61: cv1 -> m.0 -> m.1, cv2, cv3(cat[m.1 out, cv2 out])
  void c3k_inner(const std::string& pre, V x, V y, int c, bool shortcut) {
    const int ch = (int)(c * 0.5f);
    V cat = alloc(H(x), W(x), 2 * ch);
    V a = alloc(H(x), W(x), ch), b = alloc(H(x), W(x), ch);
    conv(J(pre, "cv1"), x, a, 1, 1, CK_BN_SILU);
    bottleneck(J(pre, "m.0"), a, b, ch, shortcut, false);
    bottleneck(J(pre, "m.1"), b, slice(cat, 0, ch), ch, shortcut, false);
    conv(J(pre, "cv2"), x, slice(cat, ch, ch), 1, 1, CK_BN_SILU);
    conv(J(pre, "cv3"), cat, y, 1, 1, CK_BN_SILU);
  }

  // c3k2.rs:94-127 (C2f topology: cv1 into the cat buffer, blocks append slices)
  void c3k2(const std::string& pre, V x, V y, int c_out, int n, bool c3k, bool shortcut, float e) {
    const int c = (int)(c_out * e);
    V cat = alloc(H(x), W(x), (2 + n) * c);
    conv(J(pre, "cv1"), x, slice(cat, 0, 2 * c), 1, 1, CK_BN_SILU);
    V last = slice(cat, c, c);
    for (int i = 0; i < n; ++i) {
      V out = slice(cat, (2 + i) * c, c);
      const std::string p = J(pre, "m." + std::to_string(i));
      if (c3k) c3k_inner(p, last, out, c, shortcut);
      else bottleneck(p, last, out, c, shortcut, true);
      last = out;
    }
    conv(J(pre, "cv2"), cat, y, 1, 1, CK_BN_SILU);
  }

  // c2psa.rs:61-116: qkv conv_bn -> fused attention (+PE) -> proj conv_bn (+res)
  void psa_attention(const std::string& pre, V x, V y, int c, int heads, const V* res) {
    V qkv = alloc(H(x), W(x), heads * 128);
    conv(J(pre, "qkv"), x, qkv, 1, 1, CK_BN);
    V att = alloc(H(x), W(x), c);
    // PE dw conv_bn parameters live in a ConvStep that launches nothing itself
    const int pe = conv_common(J(pre, "pe"), slice(qkv, 0, c), c, 3, 1, CK_BN, true);
    Step st;
    st.type = Step::ATTN; st.conv = pe; st.a = qkv; st.b = att; st.heads = heads;
    st.branch = branch_;
    m_->steps.push_back(st);
    conv(J(pre, "proj"), att, y, 1, 1, CK_BN, res);
  }

  // c2psa.rs:123-137: b += attn(b); b += ffn.1(ffn.0(b)), in place
  void psa_block(const std::string& pre, V b, int c, int heads) {
    psa_attention(J(pre, "attn"), b, b, c, heads, &b);
    V f = alloc(H(b), W(b), 2 * c);
    conv(J(pre, "ffn.0"), b, f, 1, 1, CK_BN_SILU);
    conv(J(pre, "ffn.1"), f, b, 1, 1, CK_BN, &b);
  }

  // c2psa.rs:150-179
  void c2psa(const std::string& pre, V x, V y, int c_out, int n, float e) {
    const int c = (int)(c_out * e);
    V cat = alloc(H(x), W(x), 2 * c);
    conv(J(pre, "cv1"), x, cat, 1, 1, CK_BN_SILU);
    V b = slice(cat, c, c);
    for (int i = 0; i < n; ++i) psa_block(J(pre, "m." + std::to_string(i)), b, c, c / 64);
    conv(J(pre, "cv2"), cat, y, 1, 1, CK_BN_SILU);
  }

  // c3k2.rs:134-164 with bottleneck_psa_seq (:67-79) as the inner block
  void c3k2_psa(const std::string& pre, V x, V y, int c_out, int n, bool shortcut, float e) {
    const int c = (int)(c_out * e);
    V cat = alloc(H(x), W(x), (2 + n) * c);
    conv(J(pre, "cv1"), x, slice(cat, 0, 2 * c), 1, 1, CK_BN_SILU);
    V last = slice(cat, c, c);
    for (int i = 0; i < n; ++i) {
      V out = slice(cat, (2 + i) * c, c);
      const std::string p = J(pre, "m." + std::to_string(i));
      bottleneck(J(p, "0"), last, out, c, shortcut, true);
      psa_block(J(p, "1"), out, c, c / 64);
      last = out;
    }
    conv(J(pre, "cv2"), cat, y, 1, 1, CK_BN_SILU);
  }

  // sppf.rs:43-61: cv1 into slice 0 of a 4c buffer, pool cascade fills the rest
  void sppf(const std::string& pre, V x, V y, int c_in, int c_out, bool shortcut) {
    const int c = c_in / 2;
    V cat = alloc(H(x), W(x), 4 * c);
    conv(J(pre, "cv1"), x, slice(cat, 0, c), 1, 1, CK_BN);
    Step st;
    st.type = Step::POOL; st.a = cat;
    st.branch = branch_;
    m_->steps.push_back(st);
    const bool add = shortcut && c_in == c_out;
    conv(J(pre, "cv2"), cat, y, 1, 1, CK_BN_SILU, add ? &x : nullptr);
  }

  void upsample(V x, V y) {
    Step st;
    st.type = Step::UP; st.a = x; st.b = y;
    st.branch = branch_;
    m_->steps.push_back(st);
  }

  // detect.rs:108-172; outputs 0 (boxes) and 1 (scores) in channel_cat_flat layout
  void detect(const std::string& pre, const V feats[3], const int chs[3], int nc, bool one2one) {
    const int c2 = std::max(16, std::max(chs[0] / 4, 4));
    const int c3 = std::max(chs[0], std::min(nc, 100));
    const std::string p2 = one2one ? "one2one_cv2" : "cv2", p3 = one2one ? "one2one_cv3" : "cv3";
    int64_t A = 0;
    for (int i = 0; i < 3; ++i) A += (int64_t)H(feats[i]) * W(feats[i]);
    int64_t base = 0;
    for (int i = 0; i < 3; ++i) {
      const V x = feats[i];
      const int64_t as = (int64_t)H(x) * W(x);
      const std::string q = J(pre, p2 + "." + std::to_string(i));
      branch_ = i;   // box chain of scale i
      V t1 = alloc(H(x), W(x), c2), t2 = alloc(H(x), W(x), c2);
      conv(J(q, "0"), x, t1, 3, 1, CK_BN_SILU);
      conv(J(q, "1"), t1, t2, 3, 1, CK_BN_SILU);
      conv_flat(J(q, "2"), t2, 4, 1, CK_PLAIN, 0, 4 * base, 4 * A, 1, as);
      base += as;
    }
    base = 0;
    for (int i = 0; i < 3; ++i) {
      const V x = feats[i];
      const int64_t as = (int64_t)H(x) * W(x);
      const std::string q = J(pre, p3 + "." + std::to_string(i));
      branch_ = 3 + i;   // class chain of scale i
      V d1 = alloc(H(x), W(x), chs[i]), p1 = alloc(H(x), W(x), c3);
      V d2 = alloc(H(x), W(x), c3), pw = alloc(H(x), W(x), c3);
      dwconv(J(q, "0.0"), x, d1, 3, 1, CK_BN_SILU);
      conv(J(q, "0.1"), d1, p1, 1, 1, CK_BN_SILU);
      dwconv(J(q, "1.0"), p1, d2, 3, 1, CK_BN_SILU);
      conv(J(q, "1.1"), d2, pw, 1, 1, CK_BN_SILU);
      conv_flat(J(q, "2"), pw, nc, 1, CK_PLAIN, 1, (int64_t)nc * base, (int64_t)nc * A, 1, as);
      base += as;
    }
    branch_ = -1;
    m_->out_dims = {{m_->batch, (int32_t)(4 * A)}, {m_->batch, (int32_t)(nc * A)}};
  }

  // model.0 straight from the NCHW float32 image (no packed input buffer)
  void stem(const std::string& pre, V y) {
    const int i = conv_common(pre, V{-1, 0, 3}, y.c, 3, 2, CK_BN_SILU, false);
    m_->convs[i].y = y;
    m_->convs[i].stem = true;
    Step st;
    st.type = Step::STEM; st.conv = i;
    st.branch = branch_;
    m_->steps.push_back(st);
  }

  V input(int c_real) { return input_at(c_real, m_->in_h, m_->in_w, 0); }

  // Input tensor [batch][c_real][h][w] at float offset `off` of the model input.
  V input_at(int c_real, int h, int w, int64_t off) {
    V in = alloc(h, w, (c_real + 7) / 8 * 8);
    real_c_[in.buf] = c_real;
    Step st;
    st.type = Step::PACK; st.b = in;
    st.in_c = c_real; st.in_h = h; st.in_w = w; st.in_off = off;
    st.branch = branch_;
    m_->steps.push_back(st);
    return in;
  }

  void output(V y) {
    Step st;
    st.type = Step::UNPACK; st.a = y; st.out_idx = (int)m_->out_dims.size();
    st.branch = branch_;
    m_->steps.push_back(st);
    m_->out_dims.push_back({m_->batch, y.c, H(y), W(y)});
  }

  int real_cin(V x) const {
    if (x.buf < 0) return x.c;
    auto it = real_c_.find(x.buf);
    return (it != real_c_.end() && x.c_off == 0 && x.c == m_->bufs[x.buf].pitch) ? it->second : x.c;
  }

 private:
  void push_conv(int i) {
    Step st;
    st.type = Step::CONV; st.conv = i;
    st.branch = branch_;
    m_->steps.push_back(st);
  }
  vrs_model* m_;
  std::unordered_map<int, int> real_c_;  // input buffer -> unpadded channels
  int branch_ = -1;                      // chain tag of the steps being added
};

int round_half_away(float v) { return (int)std::floor(v + 0.5f); }

int build(vrs_model* m) {
  Builder b(m);
  const vrs_block_desc& d = m->desc;
  switch (d.kind) {
    case VRS_BLOCK_CONV: {
      V x = b.input(d.c_in);
      const bool dw = d.g > 1 && d.g == d.c_in && d.c_in == d.c_out;
      if (d.g < 1 || d.c_in % d.g || d.c_out % d.g)
        return fail(VRS_EBADSHAPE, "conv block: channels %d -> %d not divisible by groups %d", d.c_in, d.c_out, d.g);
      if (d.conv_kind == VRS_CONV_PLAIN) {
        if (d.g > 1) return fail(VRS_EUNSUPPORTED, "conv_plain is dense");
        const int ho = (m->in_h + 2 * (d.k / 2) - d.k) / d.s + 1, wo = (m->in_w + 2 * (d.k / 2) - d.k) / d.s + 1;
        if (d.s != 1) return fail(VRS_EUNSUPPORTED, "conv_plain block: stride 1 only");
        const int64_t hw = (int64_t)ho * wo;
        b.conv_flat("", x, d.c_out, d.k, CK_PLAIN, 0, 0, d.c_out * hw, 1, hw);
        m->out_dims = {{m->batch, d.c_out, ho, wo}};
        return VRS_OK;
      }
      const int kind = d.conv_kind == VRS_CONV_BN ? CK_BN : CK_BN_SILU;
      const int ho = (m->in_h + 2 * (d.k / 2) - d.k) / d.s + 1, wo = (m->in_w + 2 * (d.k / 2) - d.k) / d.s + 1;
      V y = b.alloc(ho, wo, d.c_out);
      if (dw) b.dwconv("", x, y, d.k, d.s, kind);
      else if (d.g > 1) b.gconv("", x, y, d.k, d.s, kind, d.g);
      else b.conv("", x, y, d.k, d.s, kind);
      b.output(y);
      return VRS_OK;
    }
    case VRS_BLOCK_C3K2: {
      V x = b.input(d.c_in);
      V y = b.alloc(m->in_h, m->in_w, d.c_out);
      b.c3k2("", x, y, d.c_out, d.n, d.c3k, d.shortcut, d.e);
      b.output(y);
      return VRS_OK;
    }
    case VRS_BLOCK_C3K2_PSA: {
      V x = b.input(d.c_in);
      V y = b.alloc(m->in_h, m->in_w, d.c_out);
      b.c3k2_psa("", x, y, d.c_out, d.n, d.shortcut, d.e);
      b.output(y);
      return VRS_OK;
    }
    case VRS_BLOCK_C2PSA: {
      if (d.c_in != d.c_out) return fail(VRS_EINVAL, "C2PSA requires c_in == c_out");
      V x = b.input(d.c_in);
      V y = b.alloc(m->in_h, m->in_w, d.c_out);
      b.c2psa("", x, y, d.c_out, d.n, d.e);
      b.output(y);
      return VRS_OK;
    }
    case VRS_BLOCK_SPPF: {
      V x = b.input(d.c_in);
      V y = b.alloc(m->in_h, m->in_w, d.c_out);
      b.sppf("", x, y, d.c_in, d.c_out, d.shortcut);
      b.output(y);
      return VRS_OK;
    }
    case VRS_BLOCK_PSA_ATTN: {
      if (d.heads < 1 || d.c_in != d.heads * 64) return fail(VRS_EINVAL, "psa_attention: c must be heads*64");
      V x = b.input(d.c_in);
      V y = b.alloc(m->in_h, m->in_w, d.c_in);
      b.psa_attention("", x, y, d.c_in, d.heads, nullptr);
      b.output(y);
      return VRS_OK;
    }
    case VRS_BLOCK_DETECT_BOX: {
      const int c2 = d.c_out;
      V x = b.input(d.c_in);
      V t1 = b.alloc(m->in_h, m->in_w, c2), t2 = b.alloc(m->in_h, m->in_w, c2);
      b.conv("0", x, t1, 3, 1, CK_BN_SILU);
      b.conv("1", t1, t2, 3, 1, CK_BN_SILU);
      const int64_t hw = (int64_t)m->in_h * m->in_w;
      b.conv_flat("2", t2, 4, 1, CK_PLAIN, 0, 0, 4 * hw, 1, hw);
      m->out_dims = {{m->batch, 4, m->in_h, m->in_w}};
      return VRS_OK;
    }
    case VRS_BLOCK_DETECT: {
      // detect::<D>(nc, &ch, head) (blocks/detect.rs:108-172): the three
      // feature maps at h x w, h/2 x w/2 and h/4 x w/4 (strides 8/16/32 of the
      // image), back to back in the model input
      if (d.nc < 1) return fail(VRS_EINVAL, "detect block: nc %d", d.nc);
      if (d.ch[0] != d.c_in) return fail(VRS_EINVAL, "detect block: c_in must equal ch[0]");
      if (m->in_h % 4 || m->in_w % 4) return fail(VRS_EBADSHAPE, "detect block: h and w must be multiples of 4");
      V feats[3];
      int chs[3];
      int64_t off = 0;
      for (int i = 0; i < 3; ++i) {
        if (d.ch[i] < 1) return fail(VRS_EINVAL, "detect block: ch[%d] = %d", i, d.ch[i]);
        chs[i] = d.ch[i];
        const int hi = m->in_h >> i, wi = m->in_w >> i;
        feats[i] = b.input_at(chs[i], hi, wi, off);
        off += (int64_t)m->batch * chs[i] * hi * wi;
      }
      b.detect("", feats, chs, d.nc, d.one2one != 0);
      return VRS_OK;
    }
    case VRS_BLOCK_YOLO26: {
      float dep, wid;
      int mc;
      switch (d.variant) {  // yolo26/mod.rs:70-100
        case 'n': dep = 0.5f; wid = 0.25f; mc = 1024; break;
        case 's': dep = 0.5f; wid = 0.50f; mc = 1024; break;
        case 'm': dep = 0.5f; wid = 1.00f; mc = 512; break;
        case 'l': dep = 1.0f; wid = 1.00f; mc = 512; break;
        case 'x': dep = 1.0f; wid = 1.50f; mc = 512; break;
        default: return fail(VRS_EINVAL, "yolo26: unknown variant '%c'", (char)d.variant);
      }
      if (m->in_h % 32 || m->in_w % 32) return fail(VRS_EBADSHAPE, "yolo26: input must be divisible by 32");
      if (d.c_in != 3) return fail(VRS_EINVAL, "yolo26: 3 input channels");
      auto ch = [&](int base) { return round_half_away((float)std::min(base, mc) * wid); };  // mod.rs:106-108
      const int c0 = ch(64), c1 = ch(128), c2 = ch(256), c3 = ch(512), c4 = ch(1024);
      const int n = round_half_away(std::max(2 * dep, 1.0f));  // rep(2, d), mod.rs:111-117
      const int H = m->in_h, W = m->in_w;
      V x0 = b.alloc(H / 2, W / 2, c0);
      b.stem("model.0", x0);
      V x1 = b.alloc(H / 4, W / 4, c1);
      b.conv("model.1", x0, x1, 3, 2, CK_BN_SILU);
      V x2 = b.alloc(H / 4, W / 4, c2);
      b.c3k2("model.2", x1, x2, c2, n, false, true, 0.25f);
      V x3 = b.alloc(H / 8, W / 8, c2);
      b.conv("model.3", x2, x3, 3, 2, CK_BN_SILU);
      V cat16 = b.alloc(H / 8, W / 8, c3 + c3);       // [up(nk4), p3]
      V p3 = Builder::slice(cat16, c3, c3);
      b.c3k2("model.4", x3, p3, c3, n, false, true, 0.25f);
      V x5 = b.alloc(H / 16, W / 16, c3);
      b.conv("model.5", p3, x5, 3, 2, CK_BN_SILU);
      V cat13 = b.alloc(H / 16, W / 16, c4 + c3);     // [up(p5), p4]
      V p4 = Builder::slice(cat13, c4, c3);
      b.c3k2("model.6", x5, p4, c3, n, true, true, 0.5f);
      V x7 = b.alloc(H / 32, W / 32, c4);
      b.conv("model.7", p4, x7, 3, 2, CK_BN_SILU);
      V x8 = b.alloc(H / 32, W / 32, c4);
      b.c3k2("model.8", x7, x8, c4, n, true, true, 0.5f);
      V x9 = b.alloc(H / 32, W / 32, c4);
      b.sppf("model.9", x8, x9, c4, c4, true);
      V cat22 = b.alloc(H / 32, W / 32, c3 + c4);     // [l20(p4d), p5]
      V p5 = Builder::slice(cat22, c3, c4);
      b.c2psa("model.10", x9, p5, c4, n, 0.5f);
      b.upsample(p5, Builder::slice(cat13, 0, c4));
      V cat19 = b.alloc(H / 16, W / 16, c2 + c3);     // [l17(p3d), nk4]
      V nk4 = Builder::slice(cat19, c2, c3);
      b.c3k2("model.13", cat13, nk4, c3, n, true, true, 0.5f);
      b.upsample(nk4, Builder::slice(cat16, 0, c3));
      V p3d = b.alloc(H / 8, W / 8, c2);
      b.c3k2("model.16", cat16, p3d, c2, n, true, true, 0.5f);
      b.conv("model.17", p3d, Builder::slice(cat19, 0, c2), 3, 2, CK_BN_SILU);
      V p4d = b.alloc(H / 16, W / 16, c3);
      b.c3k2("model.19", cat19, p4d, c3, n, true, true, 0.5f);
      b.conv("model.20", p4d, Builder::slice(cat22, 0, c3), 3, 2, CK_BN_SILU);
      V p5d = b.alloc(H / 32, W / 32, c4);
      b.c3k2_psa("model.22", cat22, p5d, c4, 1, true, 0.5f);
      const V feats[3] = {p3d, p4d, p5d};
      const int chs[3] = {c2, c3, c4};
      b.detect("model.23", feats, chs, d.nc, d.one2one != 0);
      return VRS_OK;
    }
    default:
      return fail(VRS_EINVAL, "unknown block kind %d", d.kind);
  }
}

vrs_nhwc view_of(const vrs_model* m, V v) {
  const Buf& b = m->bufs[v.buf];
  vrs_nhwc r;
  r.data = b.dev; r.n = m->batch; r.h = b.h; r.w = b.w; r.c = v.c; r.pitch = b.pitch; r.c_off = v.c_off;
  return r;
}

// Conv i as the second layer of a stem pair (vrs_conv_stem_pair): it
// directly follows the stem and reads exactly the stem's output, which
// nothing else reads; 3x3 stride 2, 64 -> 128 channels, BN + SiLU on both,
// bf16 activations, image width a multiple of 4.
bool pair_eligible(const vrs_model* m, size_t i) {
  if (i == 0 || i >= m->convs.size()) return false;
  const ConvStep& s = m->convs[i - 1];
  const ConvStep& c = m->convs[i];
  if (!s.stem || s.cout != 64 || s.kind != CK_BN_SILU || s.y.buf < 0) return false;
  if (c.dw || c.groups > 1 || c.stem || c.k != 3 || c.s != 2 || c.cin != 64 || c.cout != 128 || c.kind != CK_BN_SILU || c.has_res ||
      c.has_up || c.out_idx >= 0 || c.y.buf < 0)
    return false;
  if (c.x.buf != s.y.buf || c.x.c_off != s.y.c_off || c.x.c != s.y.c) return false;
  if (act_dt(m) != VRS_BF16 || stem_pair_check(VRS_BF16, VRS_ACT_SILU, VRS_ACT_SILU, m->in_h, m->in_w) != VRS_OK) {
    (void)vrs_last_error();
    return false;
  }
  const int b = s.y.buf;
  for (size_t k = 0; k < m->convs.size(); ++k) {
    const ConvStep& o = m->convs[k];
    if (k == i || o.stem) continue;
    if (o.x.buf == b || (o.has_res && o.res.buf == b) || (o.has_up && o.up.buf == b)) return false;
  }
  for (const Step& st : m->steps)
    if ((st.type == Step::POOL || st.type == Step::UP || st.type == Step::ATTN || st.type == Step::UNPACK) &&
        st.a.buf == b)
      return false;
  return true;
}

// conv i runs as the second layer of a stem pair in this forward
bool pair_fused(const vrs_model* m, size_t i) {
  return !m->calib_mode && i < m->convs.size() && m->convs[i].tile == VRS_TILE_STEM_PAIR &&
         !(m->convs[i].f8 && m->convs[i].run_f8);
}

// Conv i as the second conv of a bottleneck pair (vrs_conv_bottleneck_pair):
// conv i-1 and conv i are 3x3 stride-1 BN + SiLU convs of a bf16 model in the
// shapes the fused kernel is built for, conv i reads exactly conv i-1's
// output, which nothing else reads or writes, and conv i's output overlaps
// neither conv i-1's input nor its own residual (the fused kernel reads those
// while other workgroups write the output).
bool bpair_eligible(const vrs_model* m, size_t i) {
  if (i == 0 || i >= m->convs.size() || m->dtype != VRS_BF16) return false;
  const ConvStep& a = m->convs[i - 1];
  const ConvStep& c = m->convs[i];
  auto plain3 = [](const ConvStep& s) {
    return !s.stem && !s.dw && s.groups <= 1 && s.k == 3 && s.s == 1 && s.kind == CK_BN_SILU && !s.has_up &&
           s.out_idx < 0 && s.x.buf >= 0 && s.y.buf >= 0 && s.cin_real == s.cin;
  };
  if (!plain3(a) || !plain3(c) || a.has_res) return false;
  if (c.x.buf != a.y.buf || c.x.c_off != a.y.c_off || c.x.c != a.y.c) return false;
  if (bpair_check(VRS_BF16, VRS_ACT_SILU, VRS_ACT_SILU, a.cin, a.cout, c.cout) != VRS_OK) {
    (void)vrs_last_error();
    return false;
  }
  auto overlap = [](V p, V q) { return p.buf == q.buf && p.c_off < q.c_off + q.c && q.c_off < p.c_off + p.c; };
  if (overlap(c.y, a.x) || (c.has_res && overlap(c.y, c.res))) return false;
  const int bb = a.y.buf;
  for (size_t k = 0; k < m->convs.size(); ++k) {
    const ConvStep& o = m->convs[k];
    if (k != i && (o.x.buf == bb || (o.has_res && o.res.buf == bb) || (o.has_up && o.up.buf == bb))) return false;
    if (k != i - 1 && o.y.buf == bb) return false;
  }
  for (const Step& st : m->steps)
    if (st.type != Step::CONV && (st.a.buf == bb || st.b.buf == bb)) return false;
  return true;
}

// conv i runs as the second conv of a bottleneck pair in this forward
bool bpair_fused(const vrs_model* m, size_t i) {
  return !m->calib_mode && i < m->convs.size() && m->convs[i].tile == VRS_TILE_BPAIR;
}

// the launch of a bottleneck pair ending at conv i
int prep_bpair_step(const vrs_model* m, size_t i, std::vector<Launch>& ls) {
  const ConvStep& a = m->convs[i - 1];
  const ConvStep& c = m->convs[i];
  vrs_nhwc r;
  if (c.has_res) r = view_of(m, c.res);
  return prep_bpair(m->ctx, view_of(m, a.x), a.w, a.scale, a.shift, a.cout, c.w, c.scale, c.shift,
                    c.has_res ? &r : nullptr, view_of(m, c.y), ls);
}

// Conv i (a Detect class output: 1x1 plain conv into a float32 flat output)
// can run fused with the 1x1 BN + SiLU conv before it as one pointwise pair:
// bf16 model, shapes the pair is built for, conv i's input exactly conv
// i-1's output, which nothing else reads or writes.
bool pwpair_eligible(const vrs_model* m, size_t i) {
  if (i == 0 || i >= m->convs.size() || m->dtype != VRS_BF16) return false;
  const ConvStep& a = m->convs[i - 1];
  const ConvStep& c = m->convs[i];
  auto plain1 = [](const ConvStep& s) {
    return !s.stem && !s.dw && s.groups <= 1 && s.k == 1 && s.s == 1 && !s.has_up && !s.has_res && s.x.buf >= 0 &&
           s.cin_real == s.cin;
  };
  if (!plain1(a) || !plain1(c) || a.kind != CK_BN_SILU || c.kind != CK_PLAIN) return false;
  if (a.out_idx >= 0 || a.y.buf < 0 || c.out_idx < 0 || c.sp < 1 || c.sc < 1) return false;
  if (c.x.buf != a.y.buf || c.x.c_off != a.y.c_off || c.x.c != a.y.c) return false;
  if (pwpair_check(VRS_BF16, VRS_ACT_SILU, VRS_ACT_NONE, a.cin, a.cout, c.cout) != VRS_OK) {
    (void)vrs_last_error();
    return false;
  }
  const int bb = a.y.buf;
  for (size_t k = 0; k < m->convs.size(); ++k) {
    const ConvStep& o = m->convs[k];
    if (k != i && (o.x.buf == bb || (o.has_res && o.res.buf == bb) || (o.has_up && o.up.buf == bb))) return false;
    if (k != i - 1 && o.y.buf == bb) return false;
  }
  for (const Step& st : m->steps)
    if (st.type != Step::CONV && (st.a.buf == bb || st.b.buf == bb)) return false;
  return true;
}

// conv i runs as the second conv of a pointwise pair in this forward
bool pwpair_fused(const vrs_model* m, size_t i) {
  return !m->calib_mode && i < m->convs.size() && m->convs[i].tile == VRS_TILE_PWPAIR;
}

// the launch of a pointwise pair ending at conv i, into outs[c.out_idx]
int prep_pwpair_step(const vrs_model* m, size_t i, float* const* outs, std::vector<Launch>& ls) {
  const ConvStep& a = m->convs[i - 1];
  const ConvStep& c = m->convs[i];
  return prep_pwpair(m->ctx, view_of(m, a.x), a.w, a.scale, a.shift, a.cout, c.w, c.scale, c.shift, c.cout,
                     outs[c.out_idx] + c.out_off, c.sb, c.sp, c.sc, ls);
}

// fp8 conv c: e4m3 input / output / residual flags and steps from the
// buffers' storage plan (steps of 1 before calibration: timing only).
void e4m3_flags(const vrs_model* m, const ConvStep& c, ConvSpec& cs) {
  auto step = [&](int b) { return m->bufs[b].step > 0.f ? m->bufs[b].step : 1.f; };
  cs.x_f8 = c.x.buf >= 0 && m->bufs[c.x.buf].f8;
  cs.y_f8 = c.out_idx < 0 && c.y.buf >= 0 && m->bufs[c.y.buf].f8;
  cs.res_f8 = c.has_res && m->bufs[c.res.buf].f8;
  if (cs.y_f8) cs.out_step = step(c.y.buf);
  if (cs.res_f8) cs.res_step = step(c.res.buf);
}

// VRS_FP8 models: the activation buffers stored as e4m3.  A buffer is when
// every launch that writes it and every conv that reads it (input, residual
// or fused-upsample source) is a conv running on the fp8 MFMA, each such
// view 16-channel aligned, and something writes it; the input and the
// fused-upsample source of one conv must agree (both e4m3, in one step group,
// or both bfloat16).  Everything else -- the stem, depthwise convs, SPPF
// pooling, attention, bf16 convs, model outputs -- keeps bfloat16 buffers.
void plan_e4m3(vrs_model* m) {
  const size_t nb = m->bufs.size();
  for (Buf& b : m->bufs) {
    b.f8 = false;
    b.grp = -1;
  }
  if (m->dtype != VRS_FP8) return;
  std::vector<char> ok(nb, 1), written(nb, 0);
  auto al16 = [&](V v) { return v.c_off % 16 == 0 && v.c % 16 == 0 && m->bufs[v.buf].pitch % 16 == 0; };
  auto no = [&](V v) { if (v.buf >= 0) ok[v.buf] = 0; };
  for (const Step& st : m->steps) {
    switch (st.type) {
      case Step::CONV: {
        const ConvStep& c = m->convs[st.conv];
        const bool f = c.f8 && c.run_f8 && !c.stem && !pair_fused(m, st.conv);
        if (pair_fused(m, st.conv)) {
          no(c.y);
          break;
        }
        for (const V* v : {&c.x, c.has_res ? &c.res : nullptr, c.has_up ? &c.up : nullptr})
          if (v && v->buf >= 0 && (!f || !al16(*v))) ok[v->buf] = 0;
        if (c.out_idx < 0 && c.y.buf >= 0) {
          written[c.y.buf] = 1;
          if (!f || !al16(c.y)) ok[c.y.buf] = 0;
        }
        break;
      }
      case Step::STEM: no(m->convs[st.conv].y); break;
      case Step::PACK: no(st.b); break;
      case Step::POOL: case Step::UNPACK: no(st.a); break;
      case Step::UP: case Step::ATTN: no(st.a); no(st.b); break;
    }
  }
  for (size_t b = 0; b < nb; ++b) m->bufs[b].f8 = ok[b] && written[b];
  // an fp8 conv's input and fused-upsample source: both e4m3 or both bf16
  for (bool changed = true; changed;) {
    changed = false;
    for (const ConvStep& c : m->convs)
      if (c.f8 && c.run_f8 && c.has_up && m->bufs[c.x.buf].f8 != m->bufs[c.up.buf].f8) {
        m->bufs[c.x.buf].f8 = m->bufs[c.up.buf].f8 = false;
        changed = true;
      }
  }
  // step groups: union of the two views of each fused-upsample conv
  std::vector<int> parent(nb);
  for (size_t b = 0; b < nb; ++b) parent[b] = (int)b;
  std::function<int(int)> root = [&](int b) { return parent[b] == b ? b : parent[b] = root(parent[b]); };
  for (const ConvStep& c : m->convs)
    if (c.f8 && c.run_f8 && c.has_up && m->bufs[c.x.buf].f8) parent[root(c.x.buf)] = root(c.up.buf);
  for (size_t b = 0; b < nb; ++b)
    if (m->bufs[b].f8) m->bufs[b].grp = root((int)b);
}

// Calibration forward (bf16): after a step that writes into a buffer planned
// as e4m3, max |x| of the written channels into the buffer's absmax slot.
int calib_writes(vrs_model* m, const LaunchIO& sio, std::vector<Launch>& ls, std::vector<std::string>& labels,
                 std::vector<LaunchIO>& io) {
  if (!m->calib_mode) return VRS_OK;
  for (const Access& w : sio.wr) {
    if (w.res < 0 || !m->bufs[w.res].f8) continue;
    vrs_nhwc v = view_of(m, V{w.res, w.c0, w.c1 - w.c0});
    const size_t before = ls.size();
    if (int rc = prep_absmax(m->ctx, v, m->absmax + m->convs.size() + w.res, ls)) return rc;
    for (size_t i = before; i < ls.size(); ++i) {
      labels.push_back("calib.buf" + std::to_string(w.res) + ":" + ls[i].name);
      io.push_back(LaunchIO{{{w.res, w.c0, w.c1}}, {}});
    }
  }
  return VRS_OK;
}

int prepare(vrs_model* m, const float* x, float* const* outs) {
  const int nout = (int)m->out_dims.size();
  std::vector<float*> o(outs, outs + nout);
  if (!m->launches.empty() && m->prep_x == x && m->prep_outs == o) return VRS_OK;
  std::vector<Launch> ls;
  std::vector<std::string> labels;
  std::vector<int> branch;
  std::vector<LaunchIO> io;
  std::vector<int> conv_launch(m->convs.size(), -1);
  int rc = VRS_OK;
  auto acc = [](V v) { return Access{v.buf, v.c_off, v.c_off + v.c}; };
  constexpr int kAll = 1 << 30;
  // a flat output conv writes [off, off + extent) of every batch row of its
  // output (the Detect scales' slices are disjoint); the whole output when
  // that range could reach the next row
  auto flat_acc = [&](const ConvStep& c) {
    const Buf& xb = m->bufs[c.x.buf];
    const int64_t ho = (xb.h + 2 * (c.k / 2) - c.k) / c.s + 1, wo = (xb.w + 2 * (c.k / 2) - c.k) / c.s + 1;
    const int64_t end = c.out_off + (ho * wo - 1) * c.sp + (int64_t)(c.cout - 1) * c.sc + 1;
    if (c.out_off < 0 || c.sp < 1 || c.sc < 1 || end > c.sb || end >= kAll) return Access{kResOut - c.out_idx, 0, kAll};
    return Access{kResOut - c.out_idx, (int)c.out_off, (int)end};
  };
  for (const Step& st : m->steps) {
    const size_t before = ls.size();
    std::string label;
    LaunchIO sio;   // this step's accesses (every launch of the step gets them)
    switch (st.type) {
      case Step::PACK: sio.rd = {{kResInput, 0, kAll}}; sio.wr = {acc(st.b)}; break;
      case Step::CONV: {
        const ConvStep& c = m->convs[st.conv];
        if (pair_fused(m, st.conv)) {   // reads the image through the fused stem
          sio.rd = {{kResInput, 0, kAll}};
          sio.wr = {acc(c.y)};
          break;
        }
        if (bpair_fused(m, st.conv)) {   // reads the first conv's input through it
          sio.rd = {acc(m->convs[st.conv - 1].x)};
          if (c.has_res) sio.rd.push_back(acc(c.res));
          sio.wr = {acc(c.y)};
          break;
        }
        sio.rd = {acc(pwpair_fused(m, st.conv) ? m->convs[st.conv - 1].x : c.x)};
        if (c.has_res) sio.rd.push_back(acc(c.res));
        if (c.has_up) sio.rd.push_back(acc(c.up));
        if (c.out_idx >= 0) sio.wr = {flat_acc(c)};
        else sio.wr = {acc(c.y)};
        break;
      }
      case Step::STEM: sio.rd = {{kResInput, 0, kAll}}; sio.wr = {acc(m->convs[st.conv].y)}; break;
      case Step::POOL: sio.rd = {acc(st.a)}; sio.wr = {acc(st.a)}; break;
      case Step::UP: case Step::ATTN: sio.rd = {acc(st.a)}; sio.wr = {acc(st.b)}; break;
      case Step::UNPACK: sio.rd = {acc(st.a)}; sio.wr = {{kResOut - st.out_idx, 0, kAll}}; break;
    }
    auto flush_io = [&]() { while (io.size() < ls.size()) io.push_back(sio); };
    switch (st.type) {
      case Step::PACK:
        rc = prep_pack_input(m->ctx, x + st.in_off, m->batch, st.in_c, st.in_h, st.in_w, view_of(m, st.b), act_dt(m),
                             ls);
        label = "input";
        break;
      case Step::CONV: {
        const ConvStep& c = m->convs[st.conv];
        if (pair_fused(m, st.conv)) {
          const ConvStep& s0 = m->convs[st.conv - 1];
          conv_launch[st.conv] = (int)ls.size();
          rc = prep_stem_pair(m->ctx, x, m->batch, m->in_h, m->in_w, s0.w, s0.scale, s0.shift, c.w, c.scale,
                              c.shift, view_of(m, c.y), ls);
          label = c.pre;
          break;
        }
        if (bpair_fused(m, st.conv + 1) || pwpair_fused(m, st.conv + 1)) continue;   // inside the next conv's launch
        if (bpair_fused(m, st.conv)) {
          conv_launch[st.conv] = (int)ls.size();
          rc = prep_bpair_step(m, st.conv, ls);
          label = c.pre;
          break;
        }
        if (pwpair_fused(m, st.conv)) {
          conv_launch[st.conv] = (int)ls.size();
          rc = prep_pwpair_step(m, st.conv, o.data(), ls);
          label = c.pre;
          break;
        }
        ConvSpec cs;
        cs.k = c.k; cs.stride = c.s; cs.dtype = act_dt(m); cs.depthwise = c.dw;
        cs.groups = c.groups;
        cs.act = c.kind == CK_BN_SILU ? VRS_ACT_SILU : VRS_ACT_NONE;
        cs.cin_real = c.cin_real != c.cin ? c.cin_real : 0;
        cs.tile = c.tile == VRS_TILE_STEM_PAIR || c.tile == VRS_TILE_PWPAIR ? VRS_TILE_AUTO : c.tile;   // unfused
        vrs_nhwc upv;
        if (c.has_up) {
          upv = view_of(m, c.up);
          cs.up = &upv;
        }
        const void* w = c.w;
        const float* scale = c.scale;
        label = c.pre.empty() ? "conv" : c.pre;
        if (c.f8 && m->calib_mode) {
          vrs_nhwc xv = view_of(m, c.x);
          if (c.has_up) {  // max |x| over the upsample source and the rest of the channels
            rc = prep_absmax(m->ctx, upv, m->absmax + st.conv, ls);
            if (rc) return rc;
            xv.c_off += c.up.c;
            xv.c -= c.up.c;
          }
          rc = prep_absmax(m->ctx, xv, m->absmax + st.conv, ls);
          if (rc) return rc;
          for (size_t i = before; i < ls.size(); ++i) labels.push_back(label + ".calib:" + ls[i].name);
        } else if (c.f8 && c.run_f8) {
          if (!m->calibrated) return fail(VRS_ESTATE, "fp8 model: call vrs_model_calibrate first");
          cs.dtype = VRS_FP8;
          cs.in_scale = c.in_scale;
          cs.tile = c.tile8;
          w = c.w8;
          scale = c.scale8;
          e4m3_flags(m, c, cs);
        }
        const size_t conv_first = ls.size();
        if (c.out_idx >= 0) {
          rc = prep_conv_flat(m->ctx, cs, view_of(m, c.x), w, scale, c.shift, c.cout, o[c.out_idx] + c.out_off,
                              c.sb, c.sp, c.sc, ls);
          // the weight-stationary float32-output tile stores 16-byte pixel
          // quads, so it needs a 16-byte aligned output slice; on a caller's
          // output that is not, the conv runs on the tiled kernel instead
          // (same results: the same K order per output)
          if (rc == VRS_EUNSUPPORTED && ((cs.tile & 0xff) == VRS_TILE_W1_128 || (cs.tile & 0xff) == VRS_TILE_W1_256)) {
            ls.resize(conv_first);
            cs.tile = VRS_TILE_AUTO;
            rc = prep_conv_flat(m->ctx, cs, view_of(m, c.x), w, scale, c.shift, c.cout, o[c.out_idx] + c.out_off,
                                c.sb, c.sp, c.sc, ls);
          }
        } else {
          vrs_nhwc r;
          if (c.has_res) r = view_of(m, c.res);
          rc = prep_conv(m->ctx, cs, view_of(m, c.x), w, scale, c.shift, c.has_res ? &r : nullptr,
                         view_of(m, c.y), ls);
        }
        if (rc) return rc;
        // the conv's output is complete after its last launch (a 256x256 conv
        // with a partial last round: full rounds, then the leftover tiles)
        conv_launch[st.conv] = (int)ls.size() - 1;
        for (size_t i = conv_first; i < ls.size(); ++i) labels.push_back(label + ":" + ls[i].name);
        flush_io();
        if ((rc = calib_writes(m, sio, ls, labels, io))) return rc;
        continue;
      }
      case Step::STEM: {
        const ConvStep& c = m->convs[st.conv];
        if (pair_fused(m, st.conv + 1)) continue;   // computed inside the next conv's launch
        conv_launch[st.conv] = (int)ls.size();
        rc = prep_stem(m->ctx, VRS_ACT_SILU, act_dt(m), x, m->batch, m->in_h, m->in_w, c.w, c.scale, c.shift,
                       c.cout, view_of(m, c.y), ls);
        label = c.pre;
        break;
      }
      case Step::POOL:
        rc = prep_pool(m->ctx, view_of(m, st.a), act_dt(m), ls);
        label = "sppf.pool";
        break;
      case Step::UP:
        rc = prep_up(m->ctx, view_of(m, st.a), view_of(m, st.b), act_dt(m), ls);
        label = "upsample";
        break;
      case Step::ATTN: {
        const ConvStep& pe = m->convs[st.conv];
        rc = prep_attn(m->ctx, st.heads, act_dt(m), view_of(m, st.a), pe.w, pe.scale,
                       pe.shift, view_of(m, st.b), ls);
        label = pe.pre.substr(0, pe.pre.size() >= 3 ? pe.pre.size() - 3 : 0) + ".core";
        break;
      }
      case Step::UNPACK:
        rc = prep_unpack(m->ctx, view_of(m, st.a), act_dt(m), o[st.out_idx], ls);
        label = "output";
        break;
    }
    if (rc) return rc;
    for (size_t i = before; i < ls.size(); ++i) labels.push_back(label + ":" + ls[i].name);
    flush_io();
    if ((rc = calib_writes(m, sio, ls, labels, io))) return rc;
    branch.resize(labels.size(), st.branch);
  }
  m->launches = std::move(ls);
  m->labels = std::move(labels);
  m->branch = std::move(branch);
  m->io = std::move(io);
  m->conv_launch = std::move(conv_launch);
  m->prep_x = x;
  m->prep_outs = o;
  return VRS_OK;
}

int dev_upload(vrs_model* m, const void* host, size_t bytes, void** dev) {
  void* p = nullptr;
  VRS_HIP(hipMalloc(&p, bytes));
  m->allocs.push_back(p);
  VRS_HIP(hipMemcpy(p, host, bytes, hipMemcpyHostToDevice));
  *dev = p;
  return VRS_OK;
}

// The convs with a tile choice (the ones a plan entry applies to): the dense
// convs, into a buffer or a Detect output.
bool tunable(const ConvStep& c) { return !c.dw && c.groups == 1 && !c.stem && (c.out_idx >= 0 || c.y.buf >= 0); }

// The launches of conv c with spec cs (tile, dtype, activation set by the
// caller) and weights w / scale: into its NHWC view, or, for a Detect output
// conv, into its channel-major float32 slice of the output tensor at `outs`.
int prep_conv_step(const vrs_model* m, const ConvStep& c, ConvSpec cs, const void* w, const float* scale,
                   float* const* outs, std::vector<Launch>& ls) {
  vrs_nhwc upv, r;
  if (c.has_up) {
    upv = view_of(m, c.up);
    cs.up = &upv;
  }
  if (c.out_idx >= 0)
    return prep_conv_flat(m->ctx, cs, view_of(m, c.x), w, scale, c.shift, c.cout, outs[c.out_idx] + c.out_off, c.sb,
                          c.sp, c.sc, ls);
  if (c.has_res) r = view_of(m, c.res);
  return prep_conv(m->ctx, cs, view_of(m, c.x), w, scale, c.shift, c.has_res ? &r : nullptr, view_of(m, c.y), ls);
}

// Time every applicable tile of each dense conv on the model's own buffers
// (contents do not matter for timing; a forward rewrites them all; the
// Detect output convs write scratch outputs) and keep the fastest.  Replaces
// the reference's shape-adaptive tile choice in TritonLowering
// (examples/yolo26.rs:3027).
int autotune_tiles(vrs_model* m) {
  hipStream_t s;
  VRS_HIP(hipStreamCreate(&s));
  hipEvent_t e0, e1;
  VRS_HIP(hipEventCreate(&e0));
  VRS_HIP(hipEventCreate(&e1));
  int rc = VRS_OK;
  // best of three rounds of five runs (every launch of the candidate): one
  // slow round (a clock dip, another process) does not decide the tile
  auto timed = [&](const std::vector<Launch>& ls, float& ms) -> int {
    ms = 1e30f;
    for (const Launch& l : ls)
      if (int r = run(l, s)) return r;
    for (int round = 0; round < 3; ++round) {
      VRS_HIP(hipEventRecord(e0, s));
      for (int it = 0; it < 5; ++it)
        for (const Launch& l : ls)
          if (int r = run(l, s)) return r;
      VRS_HIP(hipEventRecord(e1, s));
      VRS_HIP(hipEventSynchronize(e1));
      float r = 0.f;
      VRS_HIP(hipEventElapsedTime(&r, e0, e1));
      ms = std::min(ms, r);
    }
    return VRS_OK;
  };
  float* img = nullptr;   // a zero image for timing the stem pair (values do not matter)
  std::vector<float> best_bf16(m->convs.size(), 1e30f);   // each conv's fastest bf16 tile
  // scratch float32 outputs for timing the Detect output convs
  std::vector<float*> outs(m->out_dims.size(), nullptr);
  for (size_t ci = 0; ci < m->convs.size() && !rc; ++ci) {
   ConvStep& c = m->convs[ci];
   float best_of[2] = {1e30f, 1e30f};   // fastest bf16 / fp8 tile of this layer
   for (int pass = 0; pass < (c.f8 ? 2 : 1); ++pass) {
    if (!tunable(c)) continue;
    if (pass == 0 && c.f8 && m->autotune == 2) continue;   // fp8 forced: no bf16 candidates
    const int dt = pass ? VRS_FP8 : act_dt(m);
    const Buf& xb = m->bufs[c.x.buf];
    const int64_t npix = (int64_t)m->batch * ((xb.h + 2 * (c.k / 2) - c.k) / c.s + 1) *
                         ((xb.w + 2 * (c.k / 2) - c.k) / c.s + 1);
    const std::vector<int> cand =
        conv_tile_candidates(c.cout, c.cin, dt, c.k, c.s, c.has_up ? 0 : xb.w, npix, m->ctx->num_cu);
    if (cand.size() < 2) continue;
    if (c.out_idx >= 0 && !outs[c.out_idx]) {
      size_t n = 1;
      for (int32_t d : m->out_dims[c.out_idx]) n *= (size_t)d;
      if (hipMalloc(&outs[c.out_idx], n * sizeof(float)) != hipSuccess) {
        outs[c.out_idx] = nullptr;
        rc = fail(VRS_EHIP, "autotune: scratch output");
        break;
      }
    }
    ConvSpec cs;
    cs.k = c.k; cs.stride = c.s; cs.dtype = dt; cs.act = c.kind == CK_BN_SILU ? VRS_ACT_SILU : VRS_ACT_NONE;
    cs.in_scale = 1.f;  // timing only: values do not matter
    if (pass) e4m3_flags(m, c, cs);   // the storage planned for the forced fp8 model
    float best = 1e30f;
    int best_tile = VRS_TILE_AUTO;
    for (int t : cand) {
      cs.tile = t;
      std::vector<Launch> ls;
      if (prep_conv_step(m, c, cs, pass ? c.w8 : c.w, pass ? c.scale8 : c.scale, outs.data(), ls) != VRS_OK)
        continue;
      float ms;
      if ((rc = timed(ls, ms))) break;
      // a later candidate must win by 2%: near-ties keep the earlier one, so
      // the choice does not flip with timing noise from run to run
      if (ms < 0.98f * best) { best = ms; best_tile = t; }
    }
    if (rc) break;
    (pass ? c.tile8 : c.tile) = best_tile;
    best_of[pass] = best;
   }
   if (rc) break;
   // the stem pair (this conv fused with the stem before it) against this
   // conv's best tile plus the stem's own launch (forced fp8: its best fp8
   // tile -- the pair is a bf16 kernel that never writes the stem's map, and
   // runs this conv on bf16 when it wins)
   const bool forced = c.f8 && m->autotune == 2;
   const float best_alone = forced ? best_of[1] : best_of[0];
   if (pair_eligible(m, ci) && best_alone < 1e29f) {
     const ConvStep& s0 = m->convs[ci - 1];
     const size_t bytes = (size_t)m->batch * 3 * m->in_h * m->in_w * sizeof(float);
     if (!img) {
       hipError_t he = hipMalloc(&img, bytes);
       if (he == hipSuccess) he = hipMemsetAsync(img, 0, bytes, s);
       if (he != hipSuccess) {
         rc = hip_check(he, "stem pair timing image");
         break;
       }
     }
     std::vector<Launch> l0, lp;
     if (prep_stem(m->ctx, VRS_ACT_SILU, VRS_BF16, img, m->batch, m->in_h, m->in_w, s0.w, s0.scale, s0.shift,
                   s0.cout, view_of(m, s0.y), l0) == VRS_OK &&
         prep_stem_pair(m->ctx, img, m->batch, m->in_h, m->in_w, s0.w, s0.scale, s0.shift, c.w, c.scale, c.shift,
                        view_of(m, c.y), lp) == VRS_OK) {
       float t0, tp;
       if ((rc = timed(l0, t0)) || (rc = timed(lp, tp))) break;
       if (tp < 0.98f * (best_alone + t0)) {
         c.tile = VRS_TILE_STEM_PAIR;
         best_of[0] = tp - t0;
       }
     }
   }
   // a bottleneck pair (this conv fused with the 3x3 conv before it, which
   // is not itself the second conv of a pair) against the two on their own
   // fastest tiles
   best_bf16[ci] = best_of[0];
   if (bpair_eligible(m, ci) && m->convs[ci - 1].tile != VRS_TILE_BPAIR && best_of[0] < 1e29f &&
       best_bf16[ci - 1] < 1e29f) {
     std::vector<Launch> lp;
     if (prep_bpair_step(m, ci, lp) == VRS_OK) {
       float tp;
       if ((rc = timed(lp, tp))) break;
       if (tp < 0.98f * (best_of[0] + best_bf16[ci - 1])) c.tile = VRS_TILE_BPAIR;
     } else {
       (void)vrs_last_error();
     }
   }
   // a pointwise pair (this Detect class output conv fused with the 1x1 conv
   // before it) against the two on their own fastest tiles
   if (pwpair_eligible(m, ci) && best_of[0] < 1e29f && best_bf16[ci - 1] < 1e29f && outs[c.out_idx]) {
     std::vector<Launch> lp;
     if (prep_pwpair_step(m, ci, outs.data(), lp) == VRS_OK) {
       float tp;
       if ((rc = timed(lp, tp))) break;
       if (tp < 0.98f * (best_of[0] + best_bf16[ci - 1])) c.tile = VRS_TILE_PWPAIR;
     } else {
       (void)vrs_last_error();
     }
   }
   // fp8 models: a layer whose bf16 tile is faster by 2% stays on bf16
   // (unless fp8 is forced; then only the conv fused into a stem pair does)
   if (c.f8) c.run_f8 = forced ? c.tile != VRS_TILE_STEM_PAIR : !(best_of[0] < 0.98f * best_of[1]);
  }
  if (img) (void)hipFree(img);
  for (float* o : outs)
    if (o) (void)hipFree(o);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipStreamDestroy(s);
  (void)hipGetLastError();
  return rc;
}

// A nearest-2x upsample into a concat slice whose only reader is a 1x1
// stride-1 dense conv taking that slice as its first channels (the neck's
// Upsample -> Concat -> C3k2 cv1, yolo26/mod.rs:126-195) is folded into the
// conv: it reads those channels from the half-resolution source at (y/2,
// x/2), and the upsample step is dropped.
void fuse_upsamples(vrs_model* m) {
  auto overlaps = [](V a, V b) { return a.buf == b.buf && a.c_off < b.c_off + b.c && b.c_off < a.c_off + a.c; };
  for (size_t i = 0; i < m->steps.size();) {
    const Step up = m->steps[i];
    if (up.type != Step::UP) {
      ++i;
      continue;
    }
    int reader = -1, nreaders = 0;
    for (size_t j = 0; j < m->steps.size(); ++j) {
      if (j == i) continue;
      const Step& st = m->steps[j];
      std::vector<V> rd;
      if (st.type == Step::CONV) {
        const ConvStep& c = m->convs[st.conv];
        rd.push_back(c.x);
        if (c.has_res) rd.push_back(c.res);
        if (c.has_up) rd.push_back(c.up);
      } else if (st.type == Step::POOL || st.type == Step::UP || st.type == Step::ATTN || st.type == Step::UNPACK) {
        rd.push_back(st.a);
      }
      for (const V& v : rd)
        if (overlaps(v, up.b)) {
          ++nreaders;
          reader = (int)j;
          break;
        }
    }
    bool fuse = nreaders == 1 && m->steps[reader].type == Step::CONV;
    if (fuse) {
      ConvStep& c = m->convs[m->steps[reader].conv];
      fuse = !c.dw && c.groups == 1 && !c.stem && c.k == 1 && c.s == 1 && c.out_idx < 0 && c.x.buf == up.b.buf &&
             c.x.c_off == up.b.c_off && c.x.c > up.b.c && up.b.c % 64 == 0 && up.a.c == up.b.c;
      if (fuse) {
        c.up = up.a;
        c.has_up = true;
      }
    }
    if (fuse) m->steps.erase(m->steps.begin() + (ptrdiff_t)i);
    else ++i;
  }
}

const Param* P(const vrs_model* m, const std::string& name);

// Allocate the activation buffers, fold BN and upload every conv's packed
// weights and epilogue vectors (vrs_model_finalize's first step; every
// allocation is recorded in m->allocs).
int finalize_upload(vrs_model* m) {
  const size_t es = elt_size(act_dt(m));
  for (Buf& b : m->bufs) {
    const size_t bytes = (size_t)m->batch * b.h * b.w * b.pitch * es;
    VRS_HIP(hipMalloc(&b.dev, bytes));
    m->allocs.push_back(b.dev);
    VRS_HIP(hipMemset(b.dev, 0, bytes));
  }
  for (ConvStep& c : m->convs) {
    std::vector<float> scale(c.cout), shift(c.cout);
    const Param* w;
    if (c.kind == CK_PLAIN) {
      w = P(m, J(c.pre, "weight"));
      const Param* bias = P(m, J(c.pre, "bias"));
      for (int i = 0; i < c.cout; ++i) { scale[i] = 1.f; shift[i] = bias->host[i]; }
    } else {
      w = P(m, J(c.pre, "conv.weight"));
      const int rf = vrs_bn_fold(P(m, J(c.pre, "bn.weight"))->host.data(), P(m, J(c.pre, "bn.bias"))->host.data(),
                                 P(m, J(c.pre, "bn.running_mean"))->host.data(),
                                 P(m, J(c.pre, "bn.running_var"))->host.data(), m->eps, c.cout, scale.data(),
                                 shift.data());
      if (rf) return fail(rf, "%s: BN fold: %s", c.pre.c_str(), vrs_last_error());
    }
    const int cin_g = w->dims[1];
    const int groups = c.dw ? c.cout : c.groups;
    const int cin_pad = c.dw ? 1 : c.groups > 1 ? cin_g : c.cin;
    const int pdt = act_dt(m);
    const int64_t bytes = c.stem ? vrs_pack_stem_weight(nullptr, c.cout, pdt, nullptr)
                                 : vrs_pack_conv_weight(nullptr, c.cout, cin_g, c.k, groups, cin_pad, pdt, nullptr);
    if (bytes < 0) return (int)bytes;
    std::vector<uint8_t> packed((size_t)bytes);
    const int64_t r =
        c.stem ? vrs_pack_stem_weight(w->host.data(), c.cout, pdt, packed.data())
               : vrs_pack_conv_weight(w->host.data(), c.cout, cin_g, c.k, groups, cin_pad, pdt, packed.data());
    if (r < 0) return (int)r;
    int rc;
    if ((rc = dev_upload(m, packed.data(), packed.size(), &c.w))) return rc;
    void* p;
    if ((rc = dev_upload(m, scale.data(), scale.size() * 4, &p))) return rc;
    c.scale = static_cast<float*>(p);
    if ((rc = dev_upload(m, shift.data(), shift.size() * 4, &p))) return rc;
    c.shift = static_cast<float*>(p);
    c.f8 = m->dtype == VRS_FP8 && !c.dw && !c.stem && c.cin % 64 == 0 && cin_g == c.cin &&
           (!c.has_up || c.up.c % 64 == 0);
    if (c.f8) {  // e4m3 copy of the weights; the bf16 one serves calibration
      const int64_t qb = vrs_pack_conv_weight_fp8(nullptr, c.cout, cin_g, c.k, c.cin, nullptr, nullptr);
      if (qb < 0) return (int)qb;
      std::vector<uint8_t> q((size_t)qb);
      std::vector<float> ws(c.cout);
      const int64_t r8 = vrs_pack_conv_weight_fp8(w->host.data(), c.cout, cin_g, c.k, c.cin, q.data(), ws.data());
      if (r8 < 0) return (int)r8;
      if ((rc = dev_upload(m, q.data(), q.size(), &c.w8))) return rc;
      c.scale8_host.resize(c.cout);
      for (int i = 0; i < c.cout; ++i) c.scale8_host[i] = scale[i] * ws[i];
      if ((rc = dev_upload(m, c.scale8_host.data(), c.cout * 4, &p))) return rc;  // times in_scale later
      c.scale8 = static_cast<float*>(p);
    }
  }
  if (m->dtype == VRS_FP8) {
    void* p;
    VRS_HIP(hipMalloc(&p, (m->convs.size() + m->bufs.size()) * sizeof(unsigned)));
    m->allocs.push_back(p);
    m->absmax = static_cast<unsigned*>(p);
  }
  return VRS_OK;
}

// A caller's tile plan (vrs_model_set_plan) instead of autotuning: every
// entry is checked against the kernels built for its conv's shape.
int apply_plan(vrs_model* m) {
  // first the entries' kinds (which convs run on fp8 decides which buffers
  // are e4m3), then each entry validated by preparing its launch with that
  // storage
  for (size_t i = 0; i < m->convs.size(); ++i) {
    ConvStep& c = m->convs[i];
    const int32_t e = m->plan[i];
    const bool f8 = (e & VRS_PLAN_FP8) != 0;
    const int tile = e & ~VRS_PLAN_FP8;
    if (!tunable(c)) {
      if (e != 0) return fail(VRS_EINVAL, "plan entry %zu (%s): this conv takes no tile (entry must be 0)", i,
                              c.pre.c_str());
      continue;
    }
    if (f8 && !c.f8)
      return fail(VRS_EINVAL, "plan entry %zu (%s): fp8 requested for a conv that has no fp8 form", i, c.pre.c_str());
    if (tile == VRS_TILE_STEM_PAIR && (f8 || !pair_eligible(m, i)))
      return fail(VRS_EINVAL,
                  "plan entry %zu (%s): the stem pair applies only to a bf16 3x3/s2 64->128 conv reading a "
                  "64-channel stem's output alone (image width a multiple of 4)",
                  i, c.pre.c_str());
    if (tile == VRS_TILE_BPAIR &&
        (f8 || !bpair_eligible(m, i) || (m->plan[i - 1] & ~VRS_PLAN_FP8) == VRS_TILE_BPAIR))
      return fail(VRS_EINVAL,
                  "plan entry %zu (%s): the bottleneck pair applies only to the second 3x3 conv of a bf16 "
                  "bottleneck in the shapes vrs_conv_bottleneck_pair is built for, reading the first conv's output "
                  "alone, whose first conv is not itself fused as a second conv",
                  i, c.pre.c_str());
    if (tile == VRS_TILE_PWPAIR && (f8 || !pwpair_eligible(m, i)))
      return fail(VRS_EINVAL,
                  "plan entry %zu (%s): the pointwise pair applies only to a bf16 Detect class output conv in the "
                  "shapes vrs_conv_pointwise_pair is built for, reading the 1x1 conv before it alone",
                  i, c.pre.c_str());
    if (c.f8) {
      c.run_f8 = f8;
      if (f8) c.tile8 = tile;
      else c.tile = tile;
    } else {
      c.tile = tile;
    }
  }
  plan_e4m3(m);
  for (size_t i = 0; i < m->convs.size(); ++i) {
    const ConvStep& c = m->convs[i];
    const int32_t e = m->plan[i];
    const bool f8 = (e & VRS_PLAN_FP8) != 0;
    const int tile = e & ~VRS_PLAN_FP8;
    if (!tunable(c) || tile == VRS_TILE_STEM_PAIR || tile == VRS_TILE_AUTO) continue;
    if (tile == VRS_TILE_BPAIR) {   // validate by preparing the fused launch (nothing is launched)
      std::vector<Launch> ls;
      if (const int rc = prep_bpair_step(m, i, ls)) return fail(rc, "plan entry %zu (%s): %s", i, c.pre.c_str(),
                                                                 vrs_last_error());
      continue;
    }
    // a Detect output conv is prepared against a stand-in output address
    // (16-byte aligned, as every output tensor the model is given must be):
    // preparing only builds the launch arguments, nothing is launched
    std::vector<float*> probe(m->out_dims.size(), reinterpret_cast<float*>(uintptr_t{1} << 20));
    if (tile == VRS_TILE_PWPAIR) {
      std::vector<Launch> ls;
      if (const int rc = prep_pwpair_step(m, i, probe.data(), ls))
        return fail(rc, "plan entry %zu (%s): %s", i, c.pre.c_str(), vrs_last_error());
      continue;
    }
    ConvSpec cs;   // validate by preparing the launch
    cs.k = c.k; cs.stride = c.s; cs.dtype = f8 ? VRS_FP8 : act_dt(m);
    cs.act = c.kind == CK_BN_SILU ? VRS_ACT_SILU : VRS_ACT_NONE;
    cs.in_scale = 1.f;
    cs.tile = tile;
    if (f8) e4m3_flags(m, c, cs);
    std::vector<Launch> ls;
    const int rc = prep_conv_step(m, c, cs, f8 ? c.w8 : c.w, f8 ? c.scale8 : c.scale, probe.data(), ls);
    if (rc) return fail(rc, "plan entry %zu (%s): %s", i, c.pre.c_str(), vrs_last_error());
  }
  return VRS_OK;
}

const Param* P(const vrs_model* m, const std::string& name) {
  auto it = m->pidx.find(name);
  return it == m->pidx.end() ? nullptr : &m->params[it->second];
}

}  // namespace

extern "C" {

int vrs_model_create(vrs_ctx* ctx, const vrs_block_desc* d, int32_t batch, int32_t h, int32_t w, int32_t dtype,
                     float bn_eps, vrs_model** out) {
  if (!d || !out) return fail(VRS_EINVAL, "vrs_model_create: null argument");
  *out = nullptr;
  if (batch <= 0 || h <= 0 || w <= 0) return fail(VRS_EBADSHAPE, "vrs_model_create: empty input");
  if (dtype != VRS_BF16 && dtype != VRS_F32 && dtype != VRS_FP8)
    return fail(VRS_EUNSUPPORTED, "vrs_model_create: dtype %d", dtype);
  if (d->c_in <= 0 || (d->kind != VRS_BLOCK_YOLO26 && d->kind != VRS_BLOCK_DETECT && d->c_out <= 0 &&
                       d->kind != VRS_BLOCK_PSA_ATTN))
    return fail(VRS_EINVAL, "vrs_model_create: channels");
  std::unique_ptr<vrs_model> m(new vrs_model);
  m->ctx = ctx; m->desc = *d; m->batch = batch; m->in_c = d->c_in; m->in_h = h; m->in_w = w; m->dtype = dtype;
  m->eps = bn_eps;
  int rc = build(m.get());
  if (rc) return rc;
  fuse_upsamples(m.get());
  *out = m.release();
  return VRS_OK;
}

int vrs_model_num_params(const vrs_model* m) { return m ? (int)m->params.size() : fail(VRS_EINVAL, "null model"); }

int vrs_model_param_info(const vrs_model* m, int32_t i, const char** name, int32_t* dims, int32_t* ndim) {
  if (!m || !name || !dims || !ndim) return fail(VRS_EINVAL, "vrs_model_param_info: null argument");
  if (i < 0 || i >= (int)m->params.size()) return fail(VRS_EINVAL, "vrs_model_param_info: index %d", i);
  const Param& p = m->params[i];
  *name = p.name.c_str();
  *ndim = (int32_t)p.dims.size();
  for (size_t k = 0; k < p.dims.size(); ++k) dims[k] = p.dims[k];
  return VRS_OK;
}

int vrs_model_load_param(vrs_model* m, const char* name, const float* data, int64_t numel) {
  if (!m || !name || !data) return fail(VRS_EINVAL, "vrs_model_load_param: null argument");
  if (m->finalized) return fail(VRS_ESTATE, "vrs_model_load_param: model already finalized");
  auto it = m->pidx.find(name);
  if (it == m->pidx.end()) return fail(VRS_ENOTFOUND, "unknown parameter '%s'", name);
  Param& p = m->params[it->second];
  int64_t n = 1;
  for (int d : p.dims) n *= d;
  if (n != numel) return fail(VRS_EBADSHAPE, "parameter '%s' expects %lld values, got %lld", name, (long long)n,
                               (long long)numel);
  p.host.assign(data, data + numel);
  p.loaded = true;
  return VRS_OK;
}

int vrs_model_load_safetensors(vrs_model* m, const char* path, int32_t* n_loaded, int32_t* n_missing) {
  if (!m || !path) return fail(VRS_EINVAL, "vrs_model_load_safetensors: null argument");
  if (m->finalized) return fail(VRS_ESTATE, "vrs_model_load_safetensors: model already finalized");
  StFile f;
  int rc = st_open(path, f);
  if (rc) return rc;
  int32_t loaded = 0, missing = 0;
  std::vector<float> data;
  auto ends = [](const std::string& s, const char* suf) {
    const size_t n = strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
  };
  for (const Param& p : m->params) {
    // direct name, then the reference's fallback between a fused node's
    // "X.weight" and the checkpoint's "X.conv.weight" (examples/yolo26.rs:3499-3507),
    // in both directions
    const StTensor* t = st_find(f, p.name);
    if (!t && ends(p.name, ".conv.weight"))
      t = st_find(f, p.name.substr(0, p.name.size() - strlen(".conv.weight")) + ".weight");
    else if (!t && ends(p.name, ".weight"))
      t = st_find(f, p.name.substr(0, p.name.size() - strlen(".weight")) + ".conv.weight");
    if (!t) {
      ++missing;
      continue;
    }
    int64_t n = 1;
    for (int d : p.dims) n *= d;
    if (t->numel != n)
      return fail(VRS_EBADSHAPE, "safetensors: '%s' has %lld values, parameter expects %lld", p.name.c_str(),
                  (long long)t->numel, (long long)n);
    if ((rc = st_to_f32(f, p.name, *t, data))) return rc;
    if ((rc = vrs_model_load_param(m, p.name.c_str(), data.data(), n))) return rc;
    ++loaded;
  }
  if (n_loaded) *n_loaded = loaded;
  if (n_missing) *n_missing = missing;
  return VRS_OK;
}

int vrs_model_finalize(vrs_model* m) {
  if (!m) return fail(VRS_EINVAL, "null model");
  if (!m->ctx) return fail(VRS_ESTATE, "model was created without a context (record-only)");
  if (m->finalized) return VRS_OK;
  for (const Param& p : m->params)
    if (!p.loaded) return fail(VRS_ESTATE, "parameter '%s' not loaded", p.name.c_str());
  // Everything this call allocates is released again if a later step fails,
  // and the host parameters are kept until the end, so a failed finalize
  // leaves the model as it was (a retry folds and uploads again).
  const size_t first_alloc = m->allocs.size();
  int rc = finalize_upload(m);
  // forced fp8: every eligible conv runs on fp8, so the e4m3 storage is known
  // before the tiles are timed (they are timed on it)
  if (!rc && m->plan.empty()) plan_e4m3(m);
  if (!rc) rc = m->plan.empty() ? (m->autotune ? autotune_tiles(m) : VRS_OK) : apply_plan(m);
  if (!rc) plan_e4m3(m);
  // The storage is final only now: the tiles were timed on the storage of an
  // all-fp8 model, and a buffer whose reader or writer then chose bfloat16
  // stays bfloat16, so an fp8 conv reading it drops what needs an e4m3 input
  // (128-deep steps; the 64-deep tile takes either input).
  if (!rc && m->plan.empty())
    for (ConvStep& c : m->convs)
      if (c.f8 && c.run_f8 && (c.tile8 & VRS_TILE_K128) && !(c.x.buf >= 0 && m->bufs[c.x.buf].f8))
        c.tile8 &= ~VRS_TILE_K128;
  if (rc) {
    const std::string err = vrs_last_error();
    for (size_t i = first_alloc; i < m->allocs.size(); ++i) (void)hipFree(m->allocs[i]);
    m->allocs.resize(first_alloc);
    for (Buf& b : m->bufs) {
      b.dev = nullptr;
      b.f8 = false;
      b.grp = -1;
    }
    for (ConvStep& c : m->convs) {
      c.w = c.w8 = nullptr;
      c.scale = c.shift = c.scale8 = nullptr;
      c.f8 = false;
    }
    m->absmax = nullptr;
    (void)hipGetLastError();
    return fail(rc, "%s", err.c_str());
  }
  for (Param& p : m->params) std::vector<float>().swap(p.host);
  // A fused stem pair never writes the stem's output buffer (the network's
  // largest activation: 839 MB for YOLO26m at batch 64, 640x640).  Release
  // it, unless the model is fp8, whose calibration forward runs the stem on
  // its own.
  // The middle map of a fused bottleneck or pointwise pair is never written
  // either.
  if (m->dtype != VRS_FP8)
    for (size_t i = 1; i < m->convs.size(); ++i) {
      if (!(m->convs[i].tile == VRS_TILE_STEM_PAIR && pair_eligible(m, i)) && !bpair_fused(m, i) &&
          !pwpair_fused(m, i))
        continue;
      Buf& b = m->bufs[m->convs[i - 1].y.buf];
      auto it = std::find(m->allocs.begin(), m->allocs.end(), b.dev);
      if (b.dev && it != m->allocs.end()) {
        (void)hipFree(b.dev);
        m->allocs.erase(it);
        b.dev = nullptr;
      }
    }
  m->finalized = true;
  return VRS_OK;
}

int vrs_model_set_autotune(vrs_model* m, int32_t mode) {
  if (!m) return fail(VRS_EINVAL, "null model");
  if (m->finalized) return fail(VRS_ESTATE, "vrs_model_set_autotune: model already finalized");
  if (mode < 0 || mode > 2) return fail(VRS_EINVAL, "vrs_model_set_autotune: mode %d (0, 1 or 2)", mode);
  if (mode == 2 && m->dtype != VRS_FP8) return fail(VRS_EINVAL, "vrs_model_set_autotune: mode 2 is for fp8 models");
  m->autotune = mode;
  return VRS_OK;
}

int vrs_model_set_plan(vrs_model* m, const int32_t* plan, int32_t n) {
  if (!m || (!plan && n)) return fail(VRS_EINVAL, "vrs_model_set_plan: null argument");
  if (m->finalized) return fail(VRS_ESTATE, "vrs_model_set_plan: model already finalized");
  if (n != 0 && n != (int32_t)m->convs.size())
    return fail(VRS_EINVAL, "vrs_model_set_plan: %d entries for %zu convs", n, m->convs.size());
  m->plan.assign(plan, plan + n);
  return VRS_OK;
}

int vrs_model_get_plan(const vrs_model* m, int32_t* plan, int32_t n) {
  if (!m) return fail(VRS_EINVAL, "null model");
  const int32_t nc = (int32_t)m->convs.size();
  if (!plan) return nc;
  if (!m->finalized) return fail(VRS_ESTATE, "vrs_model_get_plan: call vrs_model_finalize first");
  if (n < nc) return fail(VRS_EINVAL, "vrs_model_get_plan: %d entries for %d convs", n, nc);
  for (int32_t i = 0; i < nc; ++i) {
    const ConvStep& c = m->convs[i];
    if (!tunable(c)) plan[i] = 0;
    else if (c.f8 && c.run_f8) plan[i] = c.tile8 | VRS_PLAN_FP8;
    else plan[i] = c.tile;
  }
  return nc;
}

int vrs_model_num_outputs(const vrs_model* m) { return m ? (int)m->out_dims.size() : fail(VRS_EINVAL, "null model"); }

int vrs_model_output_info(const vrs_model* m, int32_t i, int64_t* numel, int32_t* dims, int32_t* ndim) {
  if (!m || !numel || !dims || !ndim) return fail(VRS_EINVAL, "vrs_model_output_info: null argument");
  if (i < 0 || i >= (int)m->out_dims.size()) return fail(VRS_EINVAL, "vrs_model_output_info: index %d", i);
  int64_t n = 1;
  for (size_t k = 0; k < m->out_dims[i].size(); ++k) { dims[k] = m->out_dims[i][k]; n *= dims[k]; }
  *ndim = (int32_t)m->out_dims[i].size();
  *numel = n;
  return VRS_OK;
}

int vrs_model_forward(vrs_model* m, const float* x, float* const* outputs, void* stream) {
  if (!m || !x || !outputs) return fail(VRS_EINVAL, "vrs_model_forward: null argument");
  if (!m->finalized) return fail(VRS_ESTATE, "vrs_model_forward: call vrs_model_finalize first");
  for (size_t i = 0; i < m->out_dims.size(); ++i)
    if (!outputs[i]) return fail(VRS_EINVAL, "vrs_model_forward: null output %zu", i);
  int rc = prepare(m, x, outputs);
  if (rc) return rc;
  for (const Launch& l : m->launches)
    if ((rc = run(l, static_cast<hipStream_t>(stream)))) return rc;
  return VRS_OK;
}

int vrs_model_capture(vrs_model* m, const float* x, float* const* outputs, void* stream) {
  if (!m || !x || !outputs) return fail(VRS_EINVAL, "vrs_model_capture: null argument");
  if (!stream) return fail(VRS_EINVAL, "vrs_model_capture: needs a non-default stream");
  if (!m->finalized) return fail(VRS_ESTATE, "vrs_model_capture: call vrs_model_finalize first");
  int rc = prepare(m, x, outputs);
  if (rc) return rc;
  drop_graphs(m);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Concurrency: with m->streams > 1 the Detect head's chains (steps tagged
  // with a branch) may leave the caller's stream, which every other launch
  // keeps.  A chain launch continues the stream whose latest launch it
  // depends on, else (a chain starting beside others) takes the least
  // recently used stream.  Each launch waits only for the earlier launches
  // whose accesses conflict with its own -- a write against any overlapping
  // read or write of the same buffer and channel range.  All streams are
  // captured into one graph: the side streams join the capture through an
  // event recorded on the caller's stream, every cross-stream wait is a
  // captured event edge, and the side streams rejoin it before the capture
  // ends, so the graph holds the chains as parallel branches, which the
  // runtime replays on parallel hardware queues.  (Measured against the
  // alternatives: one graph per run of launches between cross-stream waits,
  // replayed on the model's streams, paid ~14 us at every graph boundary on
  // the trunk and ~50 us per replay for the fork and join; forking every
  // sibling branch of the trunk as well, and sending every chain to a side
  // stream of its own, were slower still.)
  const int n = (int)m->launches.size();
  const int K = std::max(1, std::min(m->streams, 8));
  auto conflict = [](const LaunchIO& a, const LaunchIO& b) {   // a after b
    auto ov = [](const Access& x, const Access& y) { return x.res == y.res && x.c0 < y.c1 && y.c0 < x.c1; };
    for (const Access& w : a.wr) {
      for (const Access& r : b.rd) if (ov(w, r)) return true;
      for (const Access& r : b.wr) if (ov(w, r)) return true;
    }
    for (const Access& r : a.rd)
      for (const Access& w : b.wr) if (ov(r, w)) return true;
    return false;
  };
  // stream of each launch and the cross-stream waits it needs
  std::vector<int> stream_of(n, 0), last(K, -1);
  std::vector<std::vector<int>> in_waits(n);
  std::vector<char> waited_on(n, 0);
  std::vector<std::vector<int>> waited(K, std::vector<int>(K, -1));   // [s][t]: launches of t that s has waited for
  for (int i = 0; i < n; ++i) {
    std::vector<int> deps;
    for (int j = 0; j < i; ++j)
      if (conflict(m->io[i], m->io[j])) deps.push_back(j);
    int st = 0;
    if (K > 1 && m->branch[i] >= 0) {
      st = -1;
      for (int k = 0; k < K; ++k)
        if (last[k] >= 0 && std::binary_search(deps.begin(), deps.end(), last[k]) && (st < 0 || last[k] > last[st]))
          st = k;
      if (st < 0) {
        st = 0;
        for (int k = 1; k < K; ++k) if (last[k] < last[st]) st = k;
      }
    }
    for (int j : deps) {
      const int t = stream_of[j];
      if (t == st || waited[st][t] >= j) continue;
      in_waits[i].push_back(j);
      waited_on[j] = 1;
      waited[st][t] = j;
    }
    stream_of[i] = st;
    last[st] = i;
  }
  int used = 1;
  for (int i = 0; i < n; ++i) used = std::max(used, stream_of[i] + 1);
  while ((int)m->side.size() < used - 1) {
    hipStream_t t;
    VRS_HIP(hipStreamCreateWithFlags(&t, hipStreamNonBlocking));
    m->side.push_back(t);
  }
  std::vector<hipStream_t> ss(1, s);
  for (int k = 1; k < used; ++k) ss.push_back(m->side[k - 1]);
  // capture events: the fork, one per launch another stream waits for, one
  // join per side stream; they become the graph's cross-stream edges and are
  // kept as long as the graph (drop_graphs releases them after it)
  std::vector<hipEvent_t>& evs = m->cap_evs;
  auto new_ev = [&](hipEvent_t& e) {
    const hipError_t r = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (r == hipSuccess) evs.push_back(e);
    return r;
  };
  auto free_evs = [&]() {
    for (hipEvent_t e : evs) (void)hipEventDestroy(e);
    evs.clear();
  };
  hipEvent_t fork = nullptr;
  std::vector<hipEvent_t> rec(n, nullptr), join(used, nullptr);
  bool ok = new_ev(fork) == hipSuccess;
  for (int i = 0; ok && i < n; ++i) if (waited_on[i]) ok = new_ev(rec[i]) == hipSuccess;
  for (int k = 1; ok && k < used; ++k) ok = new_ev(join[k]) == hipSuccess;
  if (!ok) {
    free_evs();
    return fail(VRS_EHIP, "vrs_model_capture: event creation failed");
  }
  if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    free_evs();
    return fail(VRS_EHIP, "vrs_model_capture: hipStreamBeginCapture failed");
  }
  const char* what = nullptr;
  if (used > 1) {
    if (hipEventRecord(fork, s) != hipSuccess) what = "fork";
    for (int k = 1; !what && k < used; ++k)
      if (hipStreamWaitEvent(ss[k], fork, 0) != hipSuccess) what = "fork";
  }
  for (int i = 0; !what && !rc && i < n; ++i) {
    const hipStream_t t = ss[stream_of[i]];
    for (int j : in_waits[i])
      if (hipStreamWaitEvent(t, rec[j], 0) != hipSuccess) what = "cross-stream wait";
    if (what || (rc = run(m->launches[i], t))) break;
    if (waited_on[i] && hipEventRecord(rec[i], t) != hipSuccess) what = "event record";
  }
  // the side streams rejoin the capture in every case, so that it can end
  for (int k = 1; k < used; ++k) {
    (void)hipEventRecord(join[k], ss[k]);
    (void)hipStreamWaitEvent(s, join[k], 0);
  }
  hipGraph_t gr = nullptr;
  const hipError_t end = hipStreamEndCapture(s, &gr);
  if (rc || what || end != hipSuccess || !gr) {
    if (gr) (void)hipGraphDestroy(gr);
    free_evs();
    if (rc) return rc;
    return fail(VRS_EHIP, "vrs_model_capture: %s", what ? what : "capture did not end");
  }
  if (hipGraphInstantiate(&m->exec, gr, nullptr, nullptr, 0) != hipSuccess) {
    (void)hipGraphDestroy(gr);
    m->exec = nullptr;
    free_evs();
    return fail(VRS_EHIP, "vrs_model_capture: graph instantiation failed");
  }
  m->graph = gr;
  m->capture_streams = used;
  return VRS_OK;
}

int vrs_model_set_streams(vrs_model* m, int32_t streams) {
  if (!m) return fail(VRS_EINVAL, "null model");
  if (streams < 1 || streams > 8) return fail(VRS_EINVAL, "vrs_model_set_streams: %d (1..8)", streams);
  m->streams = streams;
  return VRS_OK;
}

int vrs_model_replay(vrs_model* m, void* stream) {
  if (!m) return fail(VRS_EINVAL, "null model");
  if (!m->exec) return fail(VRS_ESTATE, "vrs_model_replay: no captured graph");
  VRS_HIP(hipGraphLaunch(m->exec, static_cast<hipStream_t>(stream)));
  return VRS_OK;
}

int vrs_model_num_capture_streams(const vrs_model* m) { return m && m->exec ? m->capture_streams : 0; }

int vrs_model_num_launches(const vrs_model* m) { return m ? (int)m->launches.size() : 0; }

const char* vrs_model_launch_name(const vrs_model* m, int32_t i) {
  if (!m || i < 0 || i >= (int)m->labels.size()) return "";
  return m->labels[i].c_str();
}

int vrs_model_launch_work(const vrs_model* m, int32_t i, double* flops, double* bytes) {
  if (!m || !flops || !bytes) return fail(VRS_EINVAL, "vrs_model_launch_work: null argument");
  if (i < 0 || i >= (int)m->launches.size()) return fail(VRS_EINVAL, "vrs_model_launch_work: index %d", i);
  *flops = m->launches[i].flops;
  *bytes = m->launches[i].bytes;
  return VRS_OK;
}

int vrs_model_run_launches(vrs_model* m, int32_t first, int32_t count, void* stream) {
  if (!m) return fail(VRS_EINVAL, "null model");
  if (first < 0 || count < 0 || first + count > (int)m->launches.size())
    return fail(VRS_EINVAL, "vrs_model_run_launches: range [%d,%d) of %zu", first, first + count, m->launches.size());
  for (int i = first; i < first + count; ++i) {
    int rc = run(m->launches[i], static_cast<hipStream_t>(stream));
    if (rc) return rc;
  }
  return VRS_OK;
}

int vrs_model_calibrate(vrs_model* m, const float* x, void* stream) {
  if (!m || !x) return fail(VRS_EINVAL, "vrs_model_calibrate: null argument");
  if (m->dtype != VRS_FP8) return fail(VRS_ESTATE, "vrs_model_calibrate: not an fp8 model");
  if (!m->finalized) return fail(VRS_ESTATE, "vrs_model_calibrate: call vrs_model_finalize first");
  // scratch outputs for the bf16 pass (this is set-up, not the launch path)
  std::vector<float*> outs;
  int rc = VRS_OK;
  for (const auto& d : m->out_dims) {
    int64_t n = 1;
    for (int v : d) n *= v;
    void* p = nullptr;
    if (hipMalloc(&p, (size_t)n * 4) != hipSuccess) { rc = fail(VRS_EHIP, "vrs_model_calibrate: hipMalloc"); break; }
    outs.push_back(static_cast<float*>(p));
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!rc) {
    m->calib_mode = true;
    m->launches.clear();
    m->prep_x = nullptr;
    rc = prepare(m, x, outs.data());
    if (!rc && hipMemsetAsync(m->absmax, 0, (m->convs.size() + m->bufs.size()) * sizeof(unsigned), s) != hipSuccess)
      rc = fail(VRS_EHIP, "vrs_model_calibrate: memset");
    for (size_t i = 0; !rc && i < m->launches.size(); ++i) rc = run(m->launches[i], s);
    if (!rc && hipStreamSynchronize(s) != hipSuccess) rc = fail(VRS_EHIP, "vrs_model_calibrate: sync");
  }
  std::vector<unsigned> amax(m->convs.size() + m->bufs.size());
  if (!rc && hipMemcpy(amax.data(), m->absmax, amax.size() * sizeof(unsigned), hipMemcpyDeviceToHost) != hipSuccess)
    rc = fail(VRS_EHIP, "vrs_model_calibrate: readback");
  for (float* p : outs) (void)hipFree(p);
  m->calib_mode = false;
  m->launches.clear();
  m->prep_x = nullptr;
  if (rc) return rc;
  // smallest power of two >= a / 448 (1 for an all-zero tensor)
  auto step_of = [](unsigned bits) {
    float a;
    memcpy(&a, &bits, 4);
    if (!(a > 0.f) || !std::isfinite(a)) return 1.f;
    int e;
    const float f = std::frexp(a / 448.f, &e);
    return std::ldexp(1.f, f == 0.5f ? e - 1 : e);
  };
  // e4m3 buffers: one step per group, from the largest value ever written
  // into any of its buffers
  const size_t nc = m->convs.size();
  std::vector<unsigned> gmax(m->bufs.size(), 0u);
  for (size_t b = 0; b < m->bufs.size(); ++b)
    if (m->bufs[b].f8) gmax[m->bufs[b].grp] = std::max(gmax[m->bufs[b].grp], amax[nc + b]);   // non-negative floats
  for (Buf& b : m->bufs) b.step = b.f8 ? step_of(gmax[b.grp]) : 0.f;
  for (size_t i = 0; i < nc; ++i) {
    ConvStep& c = m->convs[i];
    if (!c.f8) continue;
    // an e4m3 input is read on its buffer's step; a bf16 one is quantised on
    // the step of the conv's own input
    const float sc = m->bufs[c.x.buf].f8 ? m->bufs[c.x.buf].step : step_of(amax[i]);
    c.in_scale = sc;
    std::vector<float> s8(c.scale8_host);
    for (float& v : s8) v *= sc;
    VRS_HIP(hipMemcpy(c.scale8, s8.data(), s8.size() * 4, hipMemcpyHostToDevice));
  }
  drop_graphs(m);
  m->calibrated = true;
  return VRS_OK;
}

int vrs_model_num_convs(const vrs_model* m) { return m ? (int)m->convs.size() : fail(VRS_EINVAL, "null model"); }

int vrs_model_conv_info(const vrs_model* m, int32_t i, const char** prefix, int32_t* fp8, float* in_scale) {
  if (!m || !prefix || !fp8 || !in_scale) return fail(VRS_EINVAL, "vrs_model_conv_info: null argument");
  if (i < 0 || i >= (int)m->convs.size()) return fail(VRS_EINVAL, "vrs_model_conv_info: index %d", i);
  const ConvStep& c = m->convs[i];
  *prefix = c.pre.c_str();
  *fp8 = c.f8 && c.run_f8 ? 1 : 0;
  *in_scale = c.in_scale;
  return VRS_OK;
}

int vrs_model_conv_io(const vrs_model* m, int32_t i, vrs_conv_io* io) {
  if (!m || !io) return fail(VRS_EINVAL, "vrs_model_conv_io: null argument");
  if (i < 0 || i >= (int)m->convs.size()) return fail(VRS_EINVAL, "vrs_model_conv_io: index %d", i);
  if (!m->finalized) return fail(VRS_ESTATE, "vrs_model_conv_io: call vrs_model_finalize first");
  const ConvStep& c = m->convs[i];
  *io = vrs_conv_io{};
  io->launch = i < (int)m->conv_launch.size() ? m->conv_launch[i] : -1;
  io->k = c.k;
  io->stride = c.s;
  io->groups = c.dw ? c.cout : c.groups;
  io->act = c.kind == CK_BN_SILU ? VRS_ACT_SILU : VRS_ACT_NONE;
  io->plain = c.kind == CK_PLAIN;
  // a stem pair: the stem has no launch and no output of its own; the conv
  // after it reads the model input (stem = 2)
  // a bottleneck pair: the first conv has no launch and no output; the second
  // reads the first conv's input through it (fused_in, no x)
  // a pointwise pair likewise (the second conv writes a Detect output)
  const bool bp_out = bpair_fused(m, i + 1) || pwpair_fused(m, i + 1);
  const bool bp_in = bpair_fused(m, i) || pwpair_fused(m, i);
  const bool fused_out = (c.stem && pair_fused(m, i + 1)) || bp_out, fused_in = pair_fused(m, i);
  io->stem = fused_in ? 2 : c.stem;
  io->fused_in = fused_in || bp_in ? 1 : 0;
  io->fp8 = c.f8 && c.run_f8;
  io->in_scale = c.in_scale;
  io->dtype = act_dt(m);
  io->cin = c.cin_real;
  io->cout = c.cout;
  if (!c.stem && !fused_in && !bp_in) io->x = view_of(m, c.x);
  if (c.out_idx < 0 && c.y.buf >= 0 && !fused_out) io->y = view_of(m, c.y);
  if (c.has_res) io->res = view_of(m, c.res);
  if (c.has_up) io->up = view_of(m, c.up);
  io->out_idx = c.out_idx;
  io->out_off = c.out_off;
  io->out_sb = c.sb;
  io->out_sp = c.sp;
  io->out_sc = c.sc;
  auto e4 = [&](const vrs_nhwc& v, V src, int32_t* flag, float* step) {
    if (v.data && src.buf >= 0 && m->bufs[src.buf].f8) {
      *flag = 1;
      *step = m->bufs[src.buf].step;
    }
  };
  e4(io->x, c.x, &io->x_e4m3, &io->x_step);
  e4(io->y, c.y, &io->y_e4m3, &io->y_step);
  if (c.has_res) e4(io->res, c.res, &io->res_e4m3, &io->res_step);
  if (c.has_up) e4(io->up, c.up, &io->up_e4m3, &io->up_step);
  return VRS_OK;
}

int vrs_model_destroy(vrs_model* m) {
  if (!m) return VRS_OK;
  drop_graphs(m);
  for (hipStream_t t : m->side) (void)hipStreamDestroy(t);
  for (void* p : m->allocs) (void)hipFree(p);
  delete m;
  return VRS_OK;
}

}  // extern "C"
