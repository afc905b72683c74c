// The hidden-state VAE of the latent drafters on MI355X: TransformerHiddenVAE.encode_sequence (its
// mu) and decode_sequence (cf/vae/transformer_hidden.py:9-79), the frozen VAE that
// TreeVAEFlowDrafter runs the flow inside (cf/drafters/tree_vae_flow.py:163-175).
//
// Numerics are those of torch's fp16 modules: every Linear, LayerNorm, GELU and attention output
// is materialised in fp16 (fp32 accumulation inside), the residual stream is fp16,
// x = fp16(x + fp16(sublayer)), and nn.TransformerEncoderLayer is the pre-LN (norm_first) form
// with a GELU module after linear1 (so linear1's output is rounded before the GELU).
//
// One half (encoder or decoder) is a launch sequence on the caller's stream over the rows of one
// sequence (<= 16) -- or, for a batch, of a group of up to 128 / rows sequences stacked (the wide
// kernels of cfh_wide.h, same launches) -- built from the flow's streaming kernels (cfh_stream.h):
//   IN    stream  A = input rows                  fp32 partials                        split-K
//   RES   row     x = fp16(fp16(sum P + b_in) + pos[r]) ; a = norm1 of layer 0
//   per layer l:
//     QKV   stream  A = a                         epilogue fp16(acc + b_in)            full-K tiles
//     O     stream  A = bidirectional self attention of the k-chunk's heads            split-K by head
//     RES   row     x = fp16(x + fp16(sum P + b_o)) ; a = norm2
//     W1    stream  A = a                         epilogue fp16(gelu(fp16(acc + b1)))  full-K tiles
//     W2    stream  A = g                         fp32 partials                        split-K
//     RES   row     x = fp16(x + fp16(sum P + b2)) ; a = norm1 of layer l+1 (the final norm last)
//   OUT   stream  A = a                           fp32 partials                        split-K
//   SUM   reduce  out = fp16(sum P + b_out)
#include <algorithm>

#include "cfh_wide.h"

namespace {

// Byte offsets of one half inside the packed image.  Matrices are in MFMA tile order, vectors are
// fp16 copies of the state_dict tensors.
struct HalfLayout {
  size_t in, in_b, pos;
  size_t blk0, blkstride;
  // inside a layer
  size_t qkv, qkv_b, o, o_b, w1, w1_b, w2, w2_b, n1_w, n1_b, n2_w, n2_b;
  size_t nrm_w, nrm_b, out, out_b;
};

struct VaeLayout {
  HalfLayout enc, dec;
  size_t total;
};

bool vae_dims_ok(const cfh_vae_dims* d) {
  if (!d) return false;
  for (int v : {d->hidden, d->latent, d->inter})
    if (v <= 0 || v % 64 || v > 16384) return false;
  if (d->layers < 1 || d->layers > 16) return false;
  if (d->heads < 1 || d->inter % d->heads) return false;
  if (!cfh::heads_per_chunk(d->inter / d->heads, d->heads)) return false;
  if (d->max_rows < 1 || d->max_rows > 65536) return false;
  return true;
}

VaeLayout vae_layout(const cfh_vae_dims* dm) {
  const size_t I = dm->inter, F = 4 * I, H = 2;   // 2 bytes per element
  VaeLayout V;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = cfh::align256(off + bytes);
    return o;
  };
  auto half = [&](HalfLayout& L, size_t kin, size_t nout) {
    L.in = take(I * kin * H);
    L.in_b = take(I * H);
    L.pos = take((size_t)dm->max_rows * I * H);
    L.blk0 = off;
    size_t b = 0;
    auto btake = [&](size_t bytes) {
      const size_t o = b;
      b = cfh::align256(b + bytes);
      return o;
    };
    L.qkv = btake(3 * I * I * H);
    L.qkv_b = btake(3 * I * H);
    L.o = btake(I * I * H);
    L.o_b = btake(I * H);
    L.w1 = btake(F * I * H);
    L.w1_b = btake(F * H);
    L.w2 = btake(I * F * H);
    L.w2_b = btake(I * H);
    L.n1_w = btake(I * H);
    L.n1_b = btake(I * H);
    L.n2_w = btake(I * H);
    L.n2_b = btake(I * H);
    L.blkstride = b;
    off = L.blk0 + b * dm->layers;
    L.nrm_w = take(I * H);
    L.nrm_b = take(I * H);
    L.out = take(nout * I * H);
    L.out_b = take(nout * H);
  };
  half(V.enc, dm->hidden, dm->latent);
  half(V.dec, dm->latent, dm->hidden);
  V.total = off;
  return V;
}

struct HalfPlan {
  int Kin, Nout;
  int ks_in, wpb_in, wpb_qkv, ks_att, wpb_att, wpb_w1, ks_w2, wpb_w2, ks_out, wpb_out;
};

struct VaePlan {
  int I, F, H, hd, T;
  HalfPlan enc, dec;
  int pks, pcols;     // partial slots and their row width
  bool ok;
};

// Split-K launch shape of an N x K streaming product over T rows: as many k-chunks as reach ~2048
// wave units (at least 8 k-steps each; one chunk when K has fewer), workgroups of up to 8 waves
// that still fill one workgroup per CU.
void split_shape(int N, int K, int T, int* ks, int* wpb) {
  *ks = std::max(choose_ks(1, N / 16, K, T, 2048, 96 * 1024), 1);
  *wpb = wpb_for_grid(N / 16, *ks, 8, T * (K / *ks) / 8);
}

VaePlan vae_plan(const cfh_vae_dims* dm, int T) {
  VaePlan p = {};
  p.I = dm->inter; p.F = 4 * dm->inter; p.H = dm->heads; p.hd = p.I / p.H; p.T = T;
  const int hpk = cfh::heads_per_chunk(p.hd, p.H);
  if (!hpk) return p;
  auto half = [&](HalfPlan& h, int kin, int nout) {
    h.Kin = kin; h.Nout = nout;
    split_shape(p.I, kin, T, &h.ks_in, &h.wpb_in);
    h.wpb_qkv = wpb_for_grid(3 * p.I / 16, 1, 8, T * p.I / 8);
    h.ks_att = p.H / hpk;
    h.wpb_att = pick_wpb(p.I / 16, 1);   // (the attention staging needs the waves' slots)
    h.wpb_w1 = wpb_for_grid(p.F / 16, 1, 8, T * p.I / 8);
    split_shape(p.I, p.F, T, &h.ks_w2, &h.wpb_w2);
    split_shape(nout, p.I, T, &h.ks_out, &h.wpb_out);
  };
  half(p.enc, dm->hidden, dm->latent);
  half(p.dec, dm->latent, dm->hidden);
  p.pks = 1;
  for (const HalfPlan* h : {&p.enc, &p.dec})
    p.pks = std::max({p.pks, h->ks_in, h->ks_att, h->ks_w2, h->ks_out});
  p.pcols = std::max({p.I, dm->hidden, dm->latent});
  auto sa = [&](int N, int K, int ks, int wpb) {
    SArgs a = {};
    a.nex = 1; a.N = N; a.K = K; a.ks = ks; a.wpb = wpb; a.tpw = 1; a.d = p.I; a.hd = p.hd;
    return a;
  };
  p.ok = res_nq(p.I) > 0;
  for (const HalfPlan* h : {&p.enc, &p.dec}) {
    p.ok = p.ok && h->ks_in > 0 && h->ks_w2 > 0 && h->ks_out > 0 &&
           !stream_check(S_BUF, sa(p.I, h->Kin, h->ks_in, h->wpb_in), T) &&
           !stream_check(S_BUF, sa(3 * p.I, p.I, 1, h->wpb_qkv), T) &&
           !stream_check(S_SELF, sa(p.I, p.I, h->ks_att, h->wpb_att), T) &&
           !stream_check(S_BUF, sa(p.F, p.I, 1, h->wpb_w1), T) &&
           !stream_check(S_BUF, sa(p.I, p.F, h->ks_w2, h->wpb_w2), T) &&
           !stream_check(S_BUF, sa(h->Nout, p.I, h->ks_out, h->wpb_out), T);
  }
  return p;
}

struct VaeWS {
  float* x;      // [T][I] residual stream (fp16 values)
  h16* a;        // [T][I] LayerNorm rows
  h16* qkv;      // [T][3I]
  h16* g;        // [T][4I]
  float* P;      // [pks][T][pcols] split-K partials
  size_t total;
};

VaeWS vae_carve(const VaePlan& p, char* base) {
  VaeWS w = {};
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* q = base ? base + off : nullptr;
    off = cfh::align256(off + bytes);
    return q;
  };
  const size_t T = p.T, I = p.I;
  w.x = (float*)take(T * I * 4);
  w.a = (h16*)take(T * I * 2);
  w.qkv = (h16*)take(T * 3 * I * 2);
  w.g = (h16*)take(T * 4 * I * 2);
  w.P = (float*)take((size_t)p.pks * T * p.pcols * 4);
  w.total = off;
  return w;
}

int run_half(const VaePlan& p, const HalfPlan& hp, const HalfLayout& L, const char* W, int layers,
             const h16* in, h16* out, const VaeWS& w, hipStream_t st) {
  const int I = p.I, F = p.F, T = p.T;
  auto V = [&](size_t o) { return (const h16*)(W + o); };
  auto M = [&](size_t o) { return (const h16x8*)(W + o); };
  auto base = [&](int N, int K, int ks, int wpb) {
    SArgs a = {};
    a.nex = 1; a.N = N; a.K = K; a.ks = ks; a.wpb = wpb; a.tpw = 1; a.d = I; a.hd = p.hd;
    a.wg_per_kc = (N / 16) / wpb;
    a.ex[0].S = T;
    return a;
  };
  int rc;
  ResArgs r = {};
  r.nex = 1; r.d = I; r.x[0] = w.x; r.P[0] = w.P; r.a[0] = w.a; r.rows[0] = T;
  // IN + position rows, then norm1 of layer 0
  {
    SArgs a = base(I, hp.Kin, hp.ks_in, hp.wpb_in);
    a.ex[0].w = M(L.in); a.ex[0].a = in; a.ex[0].lda = hp.Kin; a.ex[0].out = w.P;
    if ((rc = launch_stream<S_BUF, E_PART>(a, T, st))) return rc;
    r.mode = RES_POS16; r.ks = hp.ks_in; r.bias[0] = V(L.in_b); r.pos[0] = V(L.pos);
    r.g[0] = V(L.blk0 + L.n1_w); r.b[0] = V(L.blk0 + L.n1_b);
    if ((rc = launch_res(r, st))) return rc;
  }
  r.mode = RES_ADD16;
  for (int l = 0; l < layers; ++l) {
    const size_t B = L.blk0 + (size_t)l * L.blkstride;
    {   // QKV
      SArgs a = base(3 * I, I, 1, hp.wpb_qkv);
      a.ex[0].w = M(B + L.qkv); a.ex[0].a = w.a; a.ex[0].lda = I; a.ex[0].bias = V(B + L.qkv_b);
      a.ex[0].out = w.qkv;
      if ((rc = launch_stream<S_BUF, E_BIAS16>(a, T, st))) return rc;
    }
    {   // O: bidirectional self attention, out_proj split-K by head group
      SArgs a = base(I, I, hp.ks_att, hp.wpb_att);
      a.causal = 0;
      a.ex[0].w = M(B + L.o); a.ex[0].a = w.qkv; a.ex[0].out = w.P;
      if ((rc = launch_stream<S_SELF, E_PART>(a, T, st))) return rc;
    }
    r.ks = hp.ks_att; r.bias[0] = V(B + L.o_b); r.g[0] = V(B + L.n2_w); r.b[0] = V(B + L.n2_b);
    if ((rc = launch_res(r, st))) return rc;
    {   // W1 + GELU
      SArgs a = base(F, I, 1, hp.wpb_w1);
      a.gelu_r16 = 1;
      a.ex[0].w = M(B + L.w1); a.ex[0].a = w.a; a.ex[0].lda = I; a.ex[0].bias = V(B + L.w1_b);
      a.ex[0].out = w.g;
      if ((rc = launch_stream<S_BUF, E_GELU16>(a, T, st))) return rc;
    }
    {   // W2
      SArgs a = base(I, F, hp.ks_w2, hp.wpb_w2);
      a.ex[0].w = M(B + L.w2); a.ex[0].a = w.g; a.ex[0].lda = F; a.ex[0].out = w.P;
      if ((rc = launch_stream<S_BUF, E_PART>(a, T, st))) return rc;
    }
    r.ks = hp.ks_w2; r.bias[0] = V(B + L.w2_b);
    if (l + 1 < layers) {
      r.g[0] = V(B + L.blkstride + L.n1_w); r.b[0] = V(B + L.blkstride + L.n1_b);
    } else {
      r.g[0] = V(L.nrm_w); r.b[0] = V(L.nrm_b);
    }
    if ((rc = launch_res(r, st))) return rc;
  }
  {   // OUT
    SArgs a = base(hp.Nout, I, hp.ks_out, hp.wpb_out);
    a.ex[0].w = M(L.out); a.ex[0].a = w.a; a.ex[0].lda = I; a.ex[0].out = w.P;
    if ((rc = launch_stream<S_BUF, E_PART>(a, T, st))) return rc;
    ReduceArgs ra = {};
    ra.nex = 1; ra.nl = 1; ra.ks = hp.ks_out; ra.rows = T; ra.N = hp.Nout; ra.d = hp.Nout; ra.kv = 0;
    ra.P[0] = w.P; ra.b[0] = V(L.out_b); ra.out[0] = out;
    hipLaunchKernelGGL(k_reduce, dim3(256), dim3(256), 0, st, ra);
    CFH_LAUNCH_CHECK();
  }
  return CFH_OK;
}

// Many sequences: up to WMAXR / rows of them stacked as the rows of one launch sequence through the
// wide kernels (cfh_wide.h), so that a batch of sequences streams every weight once per group
// instead of once per sequence.  Same launches and rounding points as the per-sequence form; the
// self attention runs per (sequence, head) without a mask, the position rows repeat per sequence.
struct WideHalf {
  int ks_in, wv_qkv, ks_o, wv_w1, ks_w2, ks_out;
};

struct VaeWide {
  int G, S;           // sequences a group, its rows
  WideHalf enc, dec;
  int pks, pcols;
  bool ok;
};

VaeWide vae_wide_plan(const cfh_vae_dims* dm, int rows, int G) {
  VaeWide p = {};
  const int I = dm->inter, F = 4 * I, H = dm->heads, hd = I / H;
  p.G = G;
  p.S = G * rows;
  p.pcols = std::max({I, dm->hidden, dm->latent});
  if (G < 2 || p.S > WMAXR || I % WCH || hd % 8 || (size_t)3 * rows * hd * 2 + (size_t)rows * rows * 4 > 64 * 1024)
    return p;
  constexpr int CUS = 256, WVS = 4;
  auto ks_split = [&](int N, int K) {
    int best = 0;
    for (int ks = 1; ks <= K / WCH; ++ks) {
      if (K % ks || (K / ks) % WCH) continue;
      best = ks;
      if ((long long)(N / 16 / (WT * WVS)) * ks >= CUS) break;
    }
    return best;
  };
  auto wa = [&](int N, int K, int ks) {
    WArgs a = {};
    a.nex = 1; a.N = N; a.K = K; a.ks = ks;
    return a;
  };
  p.ok = true;
  p.pks = 1;
  auto half = [&](WideHalf& h, int kin, int nout) {
    h.ks_in = kin % WCH ? 0 : ks_split(I, kin);
    h.wv_qkv = wide_wv(3 * I / 16, 1);
    h.ks_o = ks_split(I, I);
    h.wv_w1 = wide_wv(F / 16, 1);
    h.ks_w2 = ks_split(I, F);
    h.ks_out = ks_split(nout, I);
    p.ok = p.ok && h.ks_in > 0 && h.ks_o > 0 && h.ks_w2 > 0 && h.ks_out > 0 && h.wv_qkv > 0 && h.wv_w1 > 0 &&
           !wide_check(wa(I, kin, h.ks_in), WVS, p.S) && !wide_check(wa(3 * I, I, 1), h.wv_qkv, p.S) &&
           !wide_check(wa(I, I, h.ks_o), WVS, p.S) && !wide_check(wa(F, I, 1), h.wv_w1, p.S) &&
           !wide_check(wa(I, F, h.ks_w2), WVS, p.S) && !wide_check(wa(nout, I, h.ks_out), WVS, p.S);
    p.pks = std::max({p.pks, h.ks_in, h.ks_o, h.ks_w2, h.ks_out});
  };
  half(p.enc, dm->hidden, dm->latent);
  half(p.dec, dm->latent, dm->hidden);
  return p;
}

VaeWS vae_wide_carve(const VaeWide& p, const cfh_vae_dims* dm, char* base) {
  VaePlan q = {};
  q.I = dm->inter; q.T = p.S; q.pks = p.pks; q.pcols = p.pcols;
  return vae_carve(q, base);
}

int run_half_wide(const VaeWide& p, const WideHalf& hp, const HalfLayout& L, const char* W, const cfh_vae_dims* dm,
                  int rows, int G, const h16* in, h16* out, const VaeWS& w, hipStream_t st) {
  const int I = dm->inter, F = 4 * I, H = dm->heads, S = G * rows;
  const bool enc = &hp == &p.enc;
  const int Kin = enc ? dm->hidden : dm->latent, Nout = enc ? dm->latent : dm->hidden;
  auto V = [&](size_t o) { return (const h16*)(W + o); };
  auto M = [&](size_t o) { return (const h16x8*)(W + o); };
  auto one = [&](int N, int K, int ks, const h16x8* wt, const h16* a, int lda, void* o, const h16* b) {
    WArgs x = {};
    x.nex = 1; x.N = N; x.K = K; x.ks = ks;
    x.ex[0].w = wt; x.ex[0].a = a; x.ex[0].lda = lda; x.ex[0].out = o; x.ex[0].bias = b; x.ex[0].S = S;
    return x;
  };
  constexpr int WVS = 4;
  int rc;
  ResArgs r = {};
  r.nex = 1; r.d = I; r.x[0] = w.x; r.P[0] = w.P; r.a[0] = w.a; r.rows[0] = S;
  // IN + position rows (row i of the group is position i % rows of its sequence), norm1 of layer 0
  if ((rc = launch_wide<E_PART>(one(I, Kin, hp.ks_in, M(L.in), in, Kin, w.P, nullptr), WVS, st))) return rc;
  r.mode = RES_POS16; r.ks = hp.ks_in; r.bias[0] = V(L.in_b); r.pos[0] = V(L.pos); r.pos_period = rows;
  r.g[0] = V(L.blk0 + L.n1_w); r.b[0] = V(L.blk0 + L.n1_b);
  if ((rc = launch_res(r, st))) return rc;
  r.mode = RES_ADD16;
  r.pos_period = 0;
  for (int l = 0; l < dm->layers; ++l) {
    const size_t B = L.blk0 + (size_t)l * L.blkstride;
    if ((rc = launch_wide<E_BIAS16>(one(3 * I, I, 1, M(B + L.qkv), w.a, I, w.qkv, V(B + L.qkv_b)), hp.wv_qkv, st)))
      return rc;
    SelfArgs sa = {};
    sa.nex = 1; sa.R = G; sa.H = H; sa.d = I; sa.hd = I / H; sa.bidir = 1;
    sa.qkv[0] = w.qkv; sa.out[0] = w.a; sa.S[0] = S; sa.Sr[0] = rows;
    if ((rc = launch_self_attn(sa, st))) return rc;
    if ((rc = launch_wide<E_PART>(one(I, I, hp.ks_o, M(B + L.o), w.a, I, w.P, nullptr), WVS, st))) return rc;
    r.ks = hp.ks_o; r.bias[0] = V(B + L.o_b); r.g[0] = V(B + L.n2_w); r.b[0] = V(B + L.n2_b);
    if ((rc = launch_res(r, st))) return rc;
    {
      WArgs a = one(F, I, 1, M(B + L.w1), w.a, I, w.g, V(B + L.w1_b));
      a.gelu_r16 = 1;
      if ((rc = launch_wide<E_GELU16>(a, hp.wv_w1, st))) return rc;
    }
    if ((rc = launch_wide<E_PART>(one(I, F, hp.ks_w2, M(B + L.w2), w.g, F, w.P, nullptr), WVS, st))) return rc;
    r.ks = hp.ks_w2; r.bias[0] = V(B + L.w2_b);
    if (l + 1 < dm->layers) {
      r.g[0] = V(B + L.blkstride + L.n1_w); r.b[0] = V(B + L.blkstride + L.n1_b);
    } else {
      r.g[0] = V(L.nrm_w); r.b[0] = V(L.nrm_b);
    }
    if ((rc = launch_res(r, st))) return rc;
  }
  if ((rc = launch_wide<E_PART>(one(Nout, I, hp.ks_out, M(L.out), w.a, I, w.P, nullptr), WVS, st))) return rc;
  ReduceArgs ra = {};
  ra.nex = 1; ra.nl = 1; ra.ks = hp.ks_out; ra.rows = S; ra.N = Nout; ra.d = Nout; ra.kv = 0;
  ra.P[0] = w.P; ra.b[0] = V(L.out_b); ra.out[0] = out;
  hipLaunchKernelGGL(k_reduce, dim3(256), dim3(256), 0, st, ra);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// Sequences a wide group holds for `batch` sequences of `rows` rows: as few groups of at most
// WMAXR / rows as the batch needs, balanced; 1 (per-sequence launches) if the wide plan does not fit.
int vae_group(const cfh_vae_dims* dm, int rows, int batch) {
  const int gmax = WMAXR / rows;
  if (batch < 2 || gmax < 2) return 1;
  const int ng = (batch + gmax - 1) / gmax, G = (batch + ng - 1) / ng;
  return G >= 2 && vae_wide_plan(dm, rows, G).ok ? G : 1;
}

int vae_run(const cfh_vae_dims* dm, const void* packed, const void* in, void* out, int batch, int rows,
            void* ws, void* stream, bool encode) {
  if (!vae_dims_ok(dm) || rows < 1 || rows > MAXR || rows > dm->max_rows) return CFH_E_UNSUPPORTED;
  if (!packed || !in || !out || !ws || batch < 1) return CFH_E_INVALID;
  const VaePlan p = vae_plan(dm, rows);
  if (!p.ok) return CFH_E_UNSUPPORTED;
  const VaeLayout L = vae_layout(dm);
  const VaeWS w = vae_carve(p, (char*)ws);
  const HalfPlan& hp = encode ? p.enc : p.dec;
  const HalfLayout& hl = encode ? L.enc : L.dec;
  const int G = vae_group(dm, rows, batch);
  if (G > 1) {
    const VaeWide pw = vae_wide_plan(dm, rows, G);
    const VaeWS ww = vae_wide_carve(pw, dm, (char*)ws);
    for (int b0 = 0; b0 < batch; b0 += G) {
      const int g = std::min(G, batch - b0);
      const h16* ib = (const h16*)in + (size_t)b0 * rows * hp.Kin;
      h16* ob = (h16*)out + (size_t)b0 * rows * hp.Nout;
      int rc;
      if (g >= 2)
        rc = run_half_wide(pw, encode ? pw.enc : pw.dec, hl, (const char*)packed, dm, rows, g, ib, ob, ww,
                           (hipStream_t)stream);
      else
        rc = run_half(p, hp, hl, (const char*)packed, dm->layers, ib, ob, w, (hipStream_t)stream);
      if (rc) return rc;
    }
    return CFH_OK;
  }
  for (int b = 0; b < batch; ++b) {
    const h16* ib = (const h16*)in + (size_t)b * rows * hp.Kin;
    h16* ob = (h16*)out + (size_t)b * rows * hp.Nout;
    const int rc = run_half(p, hp, hl, (const char*)packed, dm->layers, ib, ob, w, (hipStream_t)stream);
    if (rc) return rc;
  }
  return CFH_OK;
}

}  // namespace

extern "C" {

int64_t cfh_vae_bytes(const cfh_vae_dims* dims) {
  if (!vae_dims_ok(dims)) return -1;
  return (int64_t)vae_layout(dims).total;
}

int cfh_vae_pack(const cfh_vae_dims* dm, const void* const* raw, int n_raw, void* packed, void* stream) {
  if (!vae_dims_ok(dm)) return CFH_E_UNSUPPORTED;
  if (!raw || !packed || n_raw != 14 + 24 * dm->layers) return CFH_E_INVALID;
  for (int i = 0; i < n_raw; ++i)
    if (!raw[i]) return CFH_E_INVALID;
  const VaeLayout V = vae_layout(dm);
  hipStream_t st = (hipStream_t)stream;
  char* base = (char*)packed;
  const size_t I = dm->inter, F = 4 * I;
  auto cp = [&](size_t off, const void* src, size_t elems) -> int {
    CFH_HIP(hipMemcpyAsync(base + off, src, elems * 2, hipMemcpyDeviceToDevice, st));
    return CFH_OK;
  };
  auto pk = [&](size_t off, const void* src, size_t n, size_t k) -> int {
    return cfh_pack_linear(src, (int)n, (int)k, base + off, stream);
  };
  int rc;
#define CFH_TRY(x) \
  if ((rc = (x)) != CFH_OK) return rc
  // one half: in.{weight,bias}, pos.weight, layers, norm.{weight,bias}, out.{weight,bias}
  auto half = [&](const HalfLayout& L, const void* const* r, size_t kin, size_t nout) -> int {
    CFH_TRY(pk(L.in, r[0], I, kin));
    CFH_TRY(cp(L.in_b, r[1], I));
    CFH_TRY(cp(L.pos, r[2], (size_t)dm->max_rows * I));
    for (int l = 0; l < dm->layers; ++l) {
      const void* const* q = r + 3 + 12 * l;
      const size_t B = L.blk0 + (size_t)l * L.blkstride;
      CFH_TRY(pk(B + L.qkv, q[0], 3 * I, I));
      CFH_TRY(cp(B + L.qkv_b, q[1], 3 * I));
      CFH_TRY(pk(B + L.o, q[2], I, I));
      CFH_TRY(cp(B + L.o_b, q[3], I));
      CFH_TRY(pk(B + L.w1, q[4], F, I));
      CFH_TRY(cp(B + L.w1_b, q[5], F));
      CFH_TRY(pk(B + L.w2, q[6], I, F));
      CFH_TRY(cp(B + L.w2_b, q[7], I));
      CFH_TRY(cp(B + L.n1_w, q[8], I));
      CFH_TRY(cp(B + L.n1_b, q[9], I));
      CFH_TRY(cp(B + L.n2_w, q[10], I));
      CFH_TRY(cp(B + L.n2_b, q[11], I));
    }
    const void* const* q = r + 3 + 12 * dm->layers;
    CFH_TRY(cp(L.nrm_w, q[0], I));
    CFH_TRY(cp(L.nrm_b, q[1], I));
    CFH_TRY(pk(L.out, q[2], nout, I));
    CFH_TRY(cp(L.out_b, q[3], nout));
    return CFH_OK;
  };
  CFH_TRY(half(V.enc, raw, dm->hidden, dm->latent));
  CFH_TRY(half(V.dec, raw + 7 + 12 * dm->layers, dm->latent, dm->hidden));
#undef CFH_TRY
  return CFH_OK;
}

int cfh_vae_caps(const cfh_vae_dims* dims, int rows, int64_t* ws_bytes) {
  if (!vae_dims_ok(dims) || rows < 1 || rows > MAXR || rows > dims->max_rows) return CFH_E_UNSUPPORTED;
  const VaePlan p = vae_plan(dims, rows);
  if (!p.ok) return CFH_E_UNSUPPORTED;
  // the per-sequence workspace, or a wide group's (every group size up to WMAXR / rows sequences)
  size_t total = vae_carve(p, nullptr).total;
  for (int G = 2; G * rows <= WMAXR; ++G) {
    const VaeWide pw = vae_wide_plan(dims, rows, G);
    if (pw.ok) total = std::max(total, vae_wide_carve(pw, dims, nullptr).total);
  }
  if (ws_bytes) *ws_bytes = (int64_t)total;
  return CFH_OK;
}

int cfh_vae_encode(const cfh_vae_dims* dims, const void* packed, const void* hidden, void* mu, int batch,
                   int rows, void* ws, void* stream) {
  return vae_run(dims, packed, hidden, mu, batch, rows, ws, stream, true);
}

int cfh_vae_decode(const cfh_vae_dims* dims, const void* packed, const void* z, void* out, int batch,
                   int rows, void* ws, void* stream) {
  return vae_run(dims, packed, z, out, batch, rows, ws, stream, false);
}

}  // extern "C"
