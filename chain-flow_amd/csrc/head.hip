// The draft head on MI355X: shortlisted lm_head (+ markov bias), per-row log-softmax top-k, the
// path-conditioned residual and the beam-search steps of the proposer.
//
// Reference semantics (cf/ = src/chain_flow/):
//   _head  = h.to(fp16) @ lm_w[sl].T -> fp16 logits      cf/vllm_plugin/flow_proposer.py:1021-1022, 739
//   _bias  = markov.w1(prev) @ markov.w2.weight[sl].T     :1024-1025, 740; cf/drafters/markov_flow.py:62-74
//   _map   = sl[local]                                     :1027-1028
//   fused path residual (one baddbmm over live offsets, masked sum, LN -> Linear -> GELU -> Linear)
//                                                          cf/vllm_plugin/fused.py:25-37
//   _beam_chains / _beam_tree depth steps and backtrack    :1187-1332
//
// The head reads the rows of the target's full lm_head in place through the int32 shortlist (a
// row-gather GEMV), so no gathered copy of lm_w[sl] is needed.
#include <limits.h>

#include "cfh_kernels.h"

namespace {

constexpr int HW = 8;       // waves per head workgroup (one 16-row vocabulary tile per wave)
constexpr int HMAXM = 8;    // max activation rows of the in-place head
constexpr int KMAX = 16;    // max top-k

// ---------------------------------------------------------------------------- head GEMV
struct HeadArgs {
  const h16* h;        // [M][d]
  const h16* W;        // [V][d]
  const int* sl;       // [n] shortlist (global row ids) or null: rows 0..n-1
  const h16* a;        // markov A: [M][r] rows, or the w1 table when a_ids is set
  const int* a_ids;    // row ids into a (a_ids[m * a_ids_stride]), or null
  const h16* W2;       // [V][r] markov w2 or null
  h16* logits;         // [M][n]
  int M, d, n, r, a_ids_stride;
};

__global__ void __launch_bounds__(HW * 64) k_head(HeadArgs a) {
  extern __shared__ __align__(16) h16 sm[];
  const int ldh = a.d + 8, ldm = a.r + 8;
  h16* Ah = sm;
  h16* Am = sm + a.M * ldh;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * HW + wave;
  const int ntiles = (a.n + 15) / 16;
  const int j = t * 16 + (lane & 15);
  const bool colv = (t < ntiles) && (j < a.n);
  const int jc = colv ? j : a.n - 1;                 // padding lanes load a valid row
  const size_t row = a.sl ? (size_t)a.sl[jc] : (size_t)jc;
  TileStream<PF, 4, false> ts;
  ts.begin((const h16x8*)(a.W + row * a.d + 8 * (lane >> 4)), a.d / 32);
  const int nh = a.d / 8;
  for (int idx = threadIdx.x; idx < a.M * nh; idx += blockDim.x) {
    const int i = idx / nh, kk = (idx - i * nh) * 8;
    *(h16x8*)(Ah + i * ldh + kk) = *(const h16x8*)(a.h + (size_t)i * a.d + kk);
  }
  if (a.W2) {
    const int nm = a.r / 8;
    for (int idx = threadIdx.x; idx < a.M * nm; idx += blockDim.x) {
      const int i = idx / nm, kk = (idx - i * nm) * 8;
      const size_t src = a.a_ids ? (size_t)max(a.a_ids[i * a.a_ids_stride], 0) : (size_t)i;
      *(h16x8*)(Am + i * ldm + kk) = *(const h16x8*)(a.a + src * a.r + kk);
    }
  }
  __syncthreads();
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = ts.run(Ah, ldh, a.M, acc);
  f32x4 accm = {0.f, 0.f, 0.f, 0.f};
  if (a.W2) {
    TileStream<PF, 4, false> tm;
    tm.begin((const h16x8*)(a.W2 + row * a.r + 8 * (lane >> 4)), a.r / 32);
    accm = tm.run(Am, ldm, a.M, accm);
  }
  if (!colv) return;
  const int rbase = 4 * (lane >> 4);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rr = rbase + q;
    if (rr < a.M) {
      const float v = a.W2 ? r16(acc[q]) + r16(accm[q]) : acc[q];
      a.logits[(size_t)rr * a.n + j] = (h16)v;
    }
  }
}

// ---------------------------------------------------------------------------- top-k
// (value, index) order: larger value first, equal values by lower index.
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

struct TopkArgs {
  const h16* logits;   // [M][ld]
  int ld, M, n, k;
  float* vals;         // [M][k] logit - logsumexp
  int* ids;            // [M][k]
  float* lse;          // [M] or null
};

// One workgroup per row: running max / sum-exp and a per-thread sorted top-KMAX list, then k
// rounds of a block-wide arg-max over the list heads.
__global__ void __launch_bounds__(1024) k_topk(TopkArgs a) {
  __shared__ float red_v[16];
  __shared__ int red_i[16];
  __shared__ float red[16];
  const int row = blockIdx.x;
  const h16* L = a.logits + (size_t)row * a.ld;
  float lv[KMAX];
  int li[KMAX];
#pragma unroll
  for (int q = 0; q < KMAX; ++q) {
    lv[q] = -INFINITY;
    li[q] = INT_MAX;
  }
  float m = -INFINITY;
  for (int i = threadIdx.x; i < a.n; i += blockDim.x) {
    const float v = (float)L[i];
    m = fmaxf(m, v);
    if (better(v, i, lv[KMAX - 1], li[KMAX - 1])) {
      lv[KMAX - 1] = v;
      li[KMAX - 1] = i;
#pragma unroll
      for (int q = KMAX - 1; q > 0; --q) {
        if (better(lv[q], li[q], lv[q - 1], li[q - 1])) {
          const float tv = lv[q]; lv[q] = lv[q - 1]; lv[q - 1] = tv;
          const int ti = li[q]; li[q] = li[q - 1]; li[q - 1] = ti;
        }
      }
    }
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  // block max
  float wm = wave_max(m);
  if (lane == 0) red[wave] = wm;
  __syncthreads();
  float mx = -INFINITY;
  for (int w = 0; w < nw; ++w) mx = fmaxf(mx, red[w]);
  __syncthreads();
  // sum of exp(v - max)
  float se = 0.f;
  for (int i = threadIdx.x; i < a.n; i += blockDim.x) se += expf((float)L[i] - mx);
  se = wave_sum(se);
  if (lane == 0) red[wave] = se;
  __syncthreads();
  float tot = 0.f;
  for (int w = 0; w < nw; ++w) tot += red[w];
  const float lse = mx + logf(tot);
  if (threadIdx.x == 0 && a.lse) a.lse[row] = lse;
  // k rounds of arg-max over the list heads
  for (int r = 0; r < a.k; ++r) {
    float bv = lv[0];
    int bi = li[0];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    __syncthreads();
    if (lane == 0) { red_v[wave] = bv; red_i[wave] = bi; }
    __syncthreads();
    bv = red_v[0];
    bi = red_i[0];
    for (int w = 1; w < nw; ++w)
      if (better(red_v[w], red_i[w], bv, bi)) { bv = red_v[w]; bi = red_i[w]; }
    if (li[0] == bi && bi != INT_MAX) {   // the owner pops its head
#pragma unroll
      for (int q = 0; q < KMAX - 1; ++q) { lv[q] = lv[q + 1]; li[q] = li[q + 1]; }
      lv[KMAX - 1] = -INFINITY;
      li[KMAX - 1] = INT_MAX;
    }
    if (threadIdx.x == 0) {
      const bool ok = bi != INT_MAX;
      a.vals[(size_t)row * a.k + r] = ok ? bv - lse : -INFINITY;
      a.ids[(size_t)row * a.k + r] = ok ? bi : -1;
    }
  }
}

// ---------------------------------------------------------------------------- path residual
struct PathSumArgs {
  const float* P;      // offset partials [o][ks][M][d]
  const h16* bias[MAXEX];
  const int* lastp;    // [M][order]
  const h16* g;        // path_head.norm weight / bias
  const h16* b;
  h16* a;              // [M][d] = fp16(LN(h))
  int order, o, ks, M, d;
};

// h = fp16(sum_j mask_j fp16(sum_kc P[j][kc] + b_j)) (the baddbmm terms, masked sum over offsets),
// then a = fp16(LN(h)).  One workgroup per row.
__global__ void __launch_bounds__(ROWT) k_path_sum(PathSumArgs a) {
  __shared__ float red[ROWT / 64];
  const int m = blockIdx.x, d = a.d, nq = d / 4;
  const size_t per_kc = (size_t)a.M * d;
  float4 vals[ROWQ];
#pragma unroll
  for (int k = 0; k < ROWQ; ++k) vals[k] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int j = 0; j < a.o; ++j) {
    if (a.lastp[m * a.order + j] < 0) continue;     // masked offset (uniform across the block)
    const float* Pj = a.P + (size_t)j * a.ks * per_kc + (size_t)m * d;
#pragma unroll
    for (int k = 0; k < ROWQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      if (q < nq) {
        float4 s4 = *(const float4*)(Pj + q * 4);
        for (int kc = 1; kc < a.ks; ++kc) {
          const float4 t = *(const float4*)(Pj + kc * per_kc + q * 4);
          s4.x += t.x; s4.y += t.y; s4.z += t.z; s4.w += t.w;
        }
        const h16* bb = a.bias[j] + q * 4;
        vals[k].x += r16(s4.x + (float)bb[0]);
        vals[k].y += r16(s4.y + (float)bb[1]);
        vals[k].z += r16(s4.z + (float)bb[2]);
        vals[k].w += r16(s4.w + (float)bb[3]);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < ROWQ; ++k) vals[k] = r16x4(vals[k]);
  ln_row4(vals, d, a.g, a.b, a.a + (size_t)m * d, red);
}

struct PathOutArgs {
  const float* P;      // down-projection partials [ks][M][d]
  const h16* bias;     // mlp.3 bias
  const h16* pred;     // [d] marginal hidden of this depth
  h16* hsum;           // [M][d] = fp16(pred + fp16(sum + b))
  int ks, M, d;
};

__global__ void __launch_bounds__(256) k_path_out(PathOutArgs a) {
  const size_t total = (size_t)a.M * a.d, per_kc = total;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int kc = 0; kc < a.ks; ++kc) s += a.P[kc * per_kc + i];
    const int c = (int)(i % a.d);
    const float res = r16(s + (float)a.bias[c]);
    a.hsum[i] = (h16)((float)a.pred[c] + res);
  }
}

struct PathPlan {
  int o_ks, up_ks, dn_ks;
  size_t off_P, off_a, off_up, off_g, off_dn, total;
};

PathPlan path_plan(int M, int d, int ffn, int order) {
  PathPlan p;
  const int pf = ffn * d;
  p.o_ks = ksplit_for(order, d / 16, d, M);
  p.up_ks = ksplit_for(1, pf / 16, d, M);
  p.dn_ks = ksplit_for(1, d / 16, pf, M);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = cfh::align256(off + bytes);
    return o;
  };
  p.off_P = take((size_t)order * p.o_ks * M * d * 4);
  p.off_a = take((size_t)M * d * 2);
  p.off_up = take((size_t)p.up_ks * M * pf * 4);
  p.off_g = take((size_t)M * pf * 2);
  p.off_dn = take((size_t)p.dn_ks * M * d * 4);
  p.total = off;
  return p;
}

// ---------------------------------------------------------------------------- beam steps
// Chain beam step (one wave per batch row, W*W <= 64): cand = cum[w] + lp[w][j];
// (cum, flat) = top-W(cand); src = flat / W; tok = sl[ids[src][flat % W]];
// lastp[w] = [tok, lastp_old[src][0 .. order-2]].
struct BeamArgs {
  const float* vals;   // [B*F][TB] per-row top-TB log-probs
  const int* ids;      // [B*F][TB] shortlist-local ids
  float* cum;          // [B][keep]: F live entries in, k out
  int* lastp;          // [B][keep][order]
  int* prev_ids;       // tree: [B][keep] node index of each frontier slot
  const int* sl;       // shortlist or null
  int* toks;           // chain: [B][W] this depth; tree: out row base pointer [B][ld_out]
  int* bps;            // chain: [B][W] parent beam; tree: parents (same row layout as toks)
  int B, F, TB, keep, order, ld_out, base;
  int tree;
};

__global__ void __launch_bounds__(64) k_beam_step(BeamArgs a) {
  __shared__ int old_lastp[64 * 8];   // F <= 64 frontier slots x order <= 8
  __shared__ int old_prev[64];
  __shared__ int win_flat[64];
  __shared__ float win_val[64];
  const int b = blockIdx.x, lane = threadIdx.x;
  const int ncand = a.F * a.TB;
  const int k = min(a.keep, ncand);
  // candidate of this lane
  float cv = -INFINITY;
  int ci = INT_MAX;
  if (lane < ncand) {
    const int f = lane / a.TB, jj = lane - f * a.TB;
    cv = a.cum[b * a.keep + f] + a.vals[((size_t)b * a.F + f) * a.TB + jj];
    ci = lane;
  }
  for (int q = lane; q < a.F * a.order; q += 64) old_lastp[q] = a.lastp[(size_t)b * a.keep * a.order + q];
  if (a.tree && lane < a.F) old_prev[lane] = a.prev_ids[b * a.keep + lane];
  __syncthreads();
  for (int r = 0; r < k; ++r) {
    float bv = cv;
    int bi = ci;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (ci == bi) { cv = -INFINITY; ci = INT_MAX; }
    if (lane == 0) { win_val[r] = bv; win_flat[r] = bi; }
  }
  __syncthreads();
  if (lane < k) {
    const int flat = win_flat[lane];
    const int src = flat / a.TB;
    const int loc = a.ids[((size_t)b * a.F + src) * a.TB + (flat - src * a.TB)];
    const int tok = loc < 0 ? -1 : (a.sl ? a.sl[loc] : loc);
    a.cum[b * a.keep + lane] = win_val[lane];
    int* lp = a.lastp + ((size_t)b * a.keep + lane) * a.order;
    lp[0] = tok;
    for (int q = 1; q < a.order; ++q) lp[q] = old_lastp[src * a.order + q - 1];
    if (a.tree) {
      a.toks[(size_t)b * a.ld_out + a.base + lane] = tok;
      a.bps[(size_t)b * a.ld_out + a.base + lane] = old_prev[src];
      a.prev_ids[b * a.keep + lane] = a.base + lane;
    } else {
      a.toks[b * a.keep + lane] = tok;
      a.bps[b * a.keep + lane] = src;
    }
  }
}

// Best chain: idx = first arg-max of cum; walk the back-pointers from the last depth.
struct BacktrackArgs {
  const float* cum;    // [B][W]
  const int* toks;     // [K][B][W]
  const int* bps;      // [K][B][W]
  long long* out;      // [B][K]
  int B, W, K;
};

__global__ void k_backtrack(BacktrackArgs a) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= a.B) return;
  int idx = 0;
  float best = a.cum[b * a.W];
  for (int w = 1; w < a.W; ++w)
    if (a.cum[b * a.W + w] > best) { best = a.cum[b * a.W + w]; idx = w; }
  for (int s = a.K - 1; s >= 0; --s) {
    const size_t o = ((size_t)s * a.B + b) * a.W + idx;
    a.out[(size_t)b * a.K + s] = a.toks[o];
    idx = a.bps[o];
  }
}

size_t head_lds(int M, int d, int r) { return (size_t)M * (d + 8) * 2 + (size_t)M * (r + 8) * 2; }

}  // namespace

extern "C" {

int cfh_head_logits(const void* h, int M, int d, const void* W, const int32_t* sl, int n, const void* a,
                    const int32_t* a_ids, int a_ids_stride, int r, const void* W2, void* logits, void* stream) {
  if (!h || !W || !logits || M < 1 || M > HMAXM || d < 32 || d % 256 || n < 1) return CFH_E_INVALID;
  if (W2 && (!a || r < 32 || r % 256)) return CFH_E_INVALID;
  HeadArgs ha = {};
  ha.h = (const h16*)h; ha.W = (const h16*)W; ha.sl = sl; ha.a = (const h16*)a; ha.a_ids = a_ids;
  ha.W2 = (const h16*)W2; ha.logits = (h16*)logits; ha.M = M; ha.d = d; ha.n = n; ha.r = W2 ? r : 0;
  ha.a_ids_stride = a_ids_stride > 0 ? a_ids_stride : 1;
  const size_t lds = head_lds(M, d, ha.r);
  if (lds > 160 * 1024) return CFH_E_UNSUPPORTED;
  CFH_HIP(hipFuncSetAttribute((const void*)k_head, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  const int ntiles = (n + 15) / 16;
  hipLaunchKernelGGL(k_head, dim3((ntiles + HW - 1) / HW), dim3(HW * 64), lds, (hipStream_t)stream, ha);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int cfh_row_topk(const void* logits, int M, int n, int k, float* vals, int32_t* ids, float* lse, void* stream) {
  if (!logits || !vals || !ids || M < 1 || n < 1 || k < 1 || k > KMAX) return CFH_E_INVALID;
  TopkArgs ta = {};
  ta.logits = (const h16*)logits; ta.ld = n; ta.M = M; ta.n = n; ta.k = k; ta.vals = vals; ta.ids = ids; ta.lse = lse;
  hipLaunchKernelGGL(k_topk, dim3(M), dim3(1024), 0, (hipStream_t)stream, ta);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int cfh_head_topk(const void* h, int M, int d, const void* W, const int32_t* sl, int n, const void* a,
                  const int32_t* a_ids, int a_ids_stride, int r, const void* W2, int k, void* logits, float* vals,
                  int32_t* ids, float* lse, void* stream) {
  int rc = cfh_head_logits(h, M, d, W, sl, n, a, a_ids, a_ids_stride, r, W2, logits, stream);
  if (rc) return rc;
  return cfh_row_topk(logits, M, n, k, vals, ids, lse, stream);
}

int64_t cfh_path_ws_bytes(int M, int d, int ffn_mult, int order) {
  if (M < 1 || M > 16 || d < 512 || d % 512 || ffn_mult < 1 || order < 1 || order > MAXEX) return -1;
  return (int64_t)path_plan(M, d, ffn_mult, order).total;
}

int cfh_path_residual(const void* const* ph, int order, int ffn_mult, int d, const int32_t* lastp, int M,
                      int nlive, const void* embed_w, const void* pred, void* hsum, void* ws, void* stream) {
  if (!ph || !lastp || !embed_w || !pred || !hsum || !ws) return CFH_E_INVALID;
  if (M < 1 || M > 16 || d < 512 || d % 512 || ffn_mult < 1 || order < 1 || order > MAXEX) return CFH_E_INVALID;
  const int n_ptr = 2 * order + 6;
  for (int i = 0; i < n_ptr; ++i)
    if (!ph[i]) return CFH_E_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const int o = (nlive < 0 || nlive > order) ? order : nlive;
  const int pf = ffn_mult * d;
  const PathPlan pp = path_plan(M, d, ffn_mult, order);
  char* base = (char*)ws;
  float* P = (float*)(base + pp.off_P);
  h16* A = (h16*)(base + pp.off_a);
  float* Pup = (float*)(base + pp.off_up);
  h16* G = (h16*)(base + pp.off_g);
  float* Pdn = (float*)(base + pp.off_dn);
  const void* const* Wj = ph;              // packed offset_proj weights
  const void* const* bj = ph + order;      // offset_proj biases
  const h16* ln_g = (const h16*)ph[2 * order];
  const h16* ln_b = (const h16*)ph[2 * order + 1];
  const h16x8* W0 = (const h16x8*)ph[2 * order + 2];
  const h16* b0 = (const h16*)ph[2 * order + 3];
  const h16x8* W3 = (const h16x8*)ph[2 * order + 4];
  const h16* b3 = (const h16*)ph[2 * order + 5];
  int rc;
  if (o > 0) {
    GemvArgs a = {};
    a.nex = o; a.nl = 1; a.ks = pp.o_ks; a.tiles = d / 16; a.N = d; a.K = d;
    for (int j = 0; j < o; ++j) {
      GemvEx& x = a.ex[j];
      x.w = (const h16x8*)Wj[j]; x.a = (const h16*)embed_w; x.lda = d; x.ids = lastp + j; x.ids_stride = order;
      x.pout = P + (size_t)j * pp.o_ks * M * d; x.rows = M;
    }
    if ((rc = launch_gemv<SRC_GATHER>(a, M, st))) return rc;
  }
  PathSumArgs ps = {};
  ps.P = P; ps.lastp = lastp; ps.g = ln_g; ps.b = ln_b; ps.a = A; ps.order = order; ps.o = o; ps.ks = pp.o_ks;
  ps.M = M; ps.d = d;
  for (int j = 0; j < o; ++j) ps.bias[j] = (const h16*)bj[j];
  hipLaunchKernelGGL(k_path_sum, dim3(M), dim3(ROWT), 0, st, ps);
  CFH_LAUNCH_CHECK();
  {
    GemvArgs a = {};
    a.nex = 1; a.nl = 1; a.ks = pp.up_ks; a.tiles = pf / 16; a.N = pf; a.K = d;
    a.ex[0].w = W0; a.ex[0].a = A; a.ex[0].lda = d; a.ex[0].pout = Pup; a.ex[0].rows = M;
    if ((rc = launch_gemv<SRC_BUF>(a, M, st))) return rc;
  }
  GeluArgs ge = {};
  ge.nex = 1; ge.ks = pp.up_ks; ge.N = pf; ge.P[0] = Pup; ge.b[0] = b0; ge.g[0] = G; ge.rows[0] = M;
  hipLaunchKernelGGL(k_gelu, dim3(64), dim3(256), 0, st, ge);
  CFH_LAUNCH_CHECK();
  {
    GemvArgs a = {};
    a.nex = 1; a.nl = 1; a.ks = pp.dn_ks; a.tiles = d / 16; a.N = d; a.K = pf;
    a.ex[0].w = W3; a.ex[0].a = G; a.ex[0].lda = pf; a.ex[0].pout = Pdn; a.ex[0].rows = M;
    if ((rc = launch_gemv<SRC_BUF>(a, M, st))) return rc;
  }
  PathOutArgs po = {};
  po.P = Pdn; po.bias = b3; po.pred = (const h16*)pred; po.hsum = (h16*)hsum; po.ks = pp.dn_ks; po.M = M; po.d = d;
  hipLaunchKernelGGL(k_path_out, dim3(64), dim3(256), 0, st, po);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int cfh_beam_chain_step(const float* vals, const int32_t* ids, float* cum, int32_t* lastp, const int32_t* sl,
                        int32_t* toks, int32_t* bps, int B, int W, int order, void* stream) {
  if (!vals || !ids || !cum || !lastp || !toks || !bps || B < 1 || W < 1 || W * W > 64 || order < 1 ||
      order > 8)
    return CFH_E_INVALID;
  BeamArgs ba = {};
  ba.vals = vals; ba.ids = ids; ba.cum = cum; ba.lastp = lastp; ba.sl = sl; ba.toks = toks; ba.bps = bps;
  ba.B = B; ba.F = W; ba.TB = W; ba.keep = W; ba.order = order; ba.tree = 0;
  hipLaunchKernelGGL(k_beam_step, dim3(B), dim3(64), 0, (hipStream_t)stream, ba);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int cfh_beam_tree_step(const float* vals, const int32_t* ids, float* cum, int32_t* lastp, int32_t* prev_ids,
                       const int32_t* sl, int32_t* out, int ld_out, int base, int B, int F, int topb, int keep,
                       int order, void* stream) {
  if (!vals || !ids || !cum || !lastp || !prev_ids || !out || B < 1 || F < 1 || F > 64 || topb < 1 ||
      F * topb > 64 || keep < 1 || keep > 64 || order < 1 || order > 8)
    return CFH_E_INVALID;
  const int k = keep < F * topb ? keep : F * topb;
  if (base + k > ld_out / 2) return CFH_E_INVALID;
  BeamArgs ba = {};
  ba.vals = vals; ba.ids = ids; ba.cum = cum; ba.lastp = lastp; ba.prev_ids = prev_ids; ba.sl = sl;
  ba.toks = out; ba.bps = out + ld_out / 2; ba.ld_out = ld_out; ba.base = base;
  ba.B = B; ba.F = F; ba.TB = topb; ba.keep = keep; ba.order = order; ba.tree = 1;
  hipLaunchKernelGGL(k_beam_step, dim3(B), dim3(64), 0, (hipStream_t)stream, ba);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int cfh_beam_backtrack(const float* cum, const int32_t* toks, const int32_t* bps, int B, int W, int K,
                       int64_t* out, void* stream) {
  if (!cum || !toks || !bps || !out || B < 1 || W < 1 || K < 1) return CFH_E_INVALID;
  BacktrackArgs ba = {};
  ba.cum = cum; ba.toks = toks; ba.bps = bps; ba.out = (long long*)out; ba.B = B; ba.W = W; ba.K = K;
  hipLaunchKernelGGL(k_backtrack, dim3((B + 63) / 64), dim3(64), 0, (hipStream_t)stream, ba);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

}  // extern "C"
