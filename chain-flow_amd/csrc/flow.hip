// The chain-flow velocity net + Euler integrator on MI355X: TreeFlowDrafter.predict_hidden.
//
// Reference semantics (cf/ = src/chain_flow/): init_latents cf/drafters/tree_flow.py:150-161,
// integrate :229-235, flow_velocity/_chunk_args :163-190, HiddenKVFlowExpert.pre_blocks /
// post_blocks cf/drafters/chunked_flow.py:333-384, HiddenKVFlowBlock.forward :185-202; fused-kernel
// numerics cf/csrc/fused_block.cu:280-325, 452-668, 674-722 (fp32 residual, fp16-parked LayerNorm
// rows, fp16 q/k/v, attention and GELU outputs, cross K/V hoisted once per draft).
//
// Execution plan: one launch sequence per draft on the caller's stream, both chunk experts in
// every launch.  Work that needs a whole row or a whole head sits at a kernel boundary; there is
// no cross-workgroup synchronisation inside any kernel (no fences, no atomics, no spin-waits), so
// every result is deterministic.
//
//   per draft : KV  (cross K/V of every block) -> REDUCE ; TAU (time_mlp(tau_s), all s) -> REDUCE ;
//               ROWS(init): z0 = init_latents(ctx), step-0 rows x, LN_self of block 0
//   per step s, per block l:
//     QKV  GEMV  A = LN_self(x)         -> fp32 partials
//     ATTN       q,k,v = fp16(sum partials + b); causal self attention -> attn (fp16)
//     O    GEMV  A = attn               -> partials
//     NORM       x += sum + b_o; A = fp16(LN_cross(fp16(x)))
//     QC   GEMV  A = LN_cross(x)        -> partials
//     ATTN       q = fp16(sum + b); attention over the hoisted context K/V -> attn
//     OC   GEMV  A = attn               -> partials
//     NORM       x += sum + b_oc; A = LN_ffn(x)
//     W1   GEMV  A = LN_ffn(x)          -> partials
//     GELU       g = fp16(gelu(sum + b1))
//     W2   GEMV  A = g                  -> partials
//     NORM       x += sum + b2; A = LN_self of the next block (out_norm after the last block)
//   OUT  GEMV  A = out_norm(x[current rows]) -> partials
//   ROWS(euler): v = fp16(sum + b_out); z = fp16(z + fp16(dt v)); next step's rows and LN_self
//
// Every GEMV is split-K over workgroups: a wave owns one (n-tile of 16 outputs, k-chunk) unit,
// streams the tile's packed fragments (cfh_common.h stream_tile) against the activation chunk held
// in LDS, and stores its fp32 partial tile; the next kernel sums the partials in chunk order.
#include <stdio.h>

#include <algorithm>
#include <mutex>

#include "cfh_kernels.h"

namespace {

// ---------------------------------------------------------------------------- attention
// One workgroup per (expert, head): softmax(q k^T / sqrt(hd) [+ causal mask]) v for <= 16 query
// rows and <= 16 keys.  q (and k, v for self attention) are reduced from the projection's fp32
// partials and rounded to fp16 as the reference materialises them; cross attention reads the
// hoisted fp16 context K/V.  Causal mask = triu(-inf, 1) (cf/drafters/chunked_flow.py:273-275).
struct AttnArgs {
  const float* P[4];   // projection partials [ks][Sq][ldp]
  const h16* bias[4];  // in_proj_bias (q at 0, k at d, v at 2d)
  const h16* kv[4];    // cross: [2][Sk][d] of this block (null for self attention)
  h16* out[4];         // [Sq][d]
  int Sq[4], Sk[4];
  int ks, ldp, d, heads, hd, causal;
};

__global__ void __launch_bounds__(1024) k_attn(AttnArgs a) {
  extern __shared__ __align__(16) h16 sm[];
  __shared__ float P[MAXR][MAXR + 1];
  const int e = blockIdx.x / a.heads, h = blockIdx.x - e * a.heads;
  const int Sq = a.Sq[e], Sk = a.Sk[e], hd = a.hd, d = a.d;
  const int c0 = h * hd;
  h16* sq = sm;
  h16* sk = sm + (size_t)Sq * hd;
  h16* sv = sk + (size_t)Sk * hd;
  const size_t pstride = (size_t)Sq * a.ldp;
  // q (and k, v) = fp16(sum of partials + bias), four columns per thread-step
  const int nsrc = a.kv[e] ? 1 : 3;
  const int hq = hd / 4;
  for (int idx = threadIdx.x; idx < nsrc * Sq * hq; idx += blockDim.x) {
    const int part = idx / (Sq * hq);
    const int r = idx - part * Sq * hq;
    const int i = r / hq, c = (r - i * hq) * 4;
    const int col = part * d + c0 + c;
    const float* Pp = a.P[e] + (size_t)i * a.ldp + col;
    float4 s4 = *(const float4*)Pp;
    for (int q = 1; q < a.ks; ++q) {
      const float4 t = *(const float4*)(Pp + q * pstride);
      s4.x += t.x; s4.y += t.y; s4.z += t.z; s4.w += t.w;
    }
    const h16* bb = a.bias[e] + col;
    h16* dst = (part == 0 ? sq : (part == 1 ? sk : sv)) + i * hd + c;
    dst[0] = (h16)(s4.x + (float)bb[0]);
    dst[1] = (h16)(s4.y + (float)bb[1]);
    dst[2] = (h16)(s4.z + (float)bb[2]);
    dst[3] = (h16)(s4.w + (float)bb[3]);
  }
  if (a.kv[e]) {
    const int nv = hd / 8;
    for (int idx = threadIdx.x; idx < Sk * nv; idx += blockDim.x) {
      const int j = idx / nv, c = (idx - j * nv) * 8;
      *(h16x8*)(sk + j * hd + c) = *(const h16x8*)(a.kv[e] + (size_t)j * d + c0 + c);
      *(h16x8*)(sv + j * hd + c) = *(const h16x8*)(a.kv[e] + (size_t)(Sk + j) * d + c0 + c);
    }
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const float scale = 1.0f / sqrtf((float)hd);
  for (int pr = wave; pr < Sq * Sk; pr += nw) {
    const int i = pr / Sk, j = pr - i * Sk;
    float part = 0.f;
    for (int c = lane * 8; c < hd; c += 512) {
      const h16x8 qa = *(const h16x8*)(sq + i * hd + c);
      const h16x8 kb = *(const h16x8*)(sk + j * hd + c);
#pragma unroll
      for (int t = 0; t < 8; ++t) part += (float)qa[t] * (float)kb[t];
    }
    const float s = wave_sum(part) * scale;
    if (lane == 0) P[i][j] = (a.causal && j > i) ? -INFINITY : s;
  }
  __syncthreads();
  if ((int)threadIdx.x < Sq) {
    const int i = threadIdx.x;
    float m = -INFINITY;
    for (int j = 0; j < Sk; ++j) m = fmaxf(m, P[i][j]);
    float den = 0.f;
    for (int j = 0; j < Sk; ++j) {
      const float ex = expf(P[i][j] - m);
      P[i][j] = ex;
      den += ex;
    }
    const float inv = 1.0f / den;
    for (int j = 0; j < Sk; ++j) P[i][j] *= inv;
  }
  __syncthreads();
  const int nv = hd / 8;
  for (int idx = threadIdx.x; idx < Sq * nv; idx += blockDim.x) {
    const int i = idx / nv, c = (idx - i * nv) * 8;
    float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < Sk; ++j) {
      const float p = P[i][j];
      const h16x8 vb = *(const h16x8*)(sv + j * hd + c);
#pragma unroll
      for (int t = 0; t < 8; ++t) o[t] += p * (float)vb[t];
    }
    h16x8 ov;
#pragma unroll
    for (int t = 0; t < 8; ++t) ov[t] = (h16)o[t];
    *(h16x8*)(a.out[e] + (size_t)i * d + c0 + c) = ov;
  }
}

// ---------------------------------------------------------------------------- row kernels
// NORM: x[r] += sum_kc P[kc][r] + bias; a[r] = fp16(LN(fp16(x[r]))).  One workgroup per row.
struct NormArgs {
  float* x[4];
  const float* P[4];
  const h16* bias[4];
  const h16* g[4];
  const h16* b[4];
  h16* a[4];
  int rows[4];
  int nex, ks, d;
};

__global__ void __launch_bounds__(ROWT) k_norm(NormArgs a) {
  __shared__ float red[ROWT / 64];
  int e = 0, r = blockIdx.x;
  while (e + 1 < a.nex && r >= a.rows[e]) r -= a.rows[e++];
  const int d = a.d, nq = d / 4;
  const size_t pst = (size_t)a.rows[e] * d;
  float* xr = a.x[e] + (size_t)r * d;
  const float* Pr = a.P[e] + (size_t)r * d;
  float4 acc[ROWQ], xv[ROWQ];
#pragma unroll
  for (int k = 0; k < ROWQ; ++k) {
    const int q = threadIdx.x + k * blockDim.x;
    if (q < nq) {
      xv[k] = *(const float4*)(xr + q * 4);
      acc[k] = *(const float4*)(Pr + q * 4);
    }
  }
#pragma unroll 4
  for (int kc = 1; kc < a.ks; ++kc) {
#pragma unroll
    for (int k = 0; k < ROWQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      if (q < nq) {
        const float4 t = *(const float4*)(Pr + kc * pst + q * 4);
        acc[k].x += t.x; acc[k].y += t.y; acc[k].z += t.z; acc[k].w += t.w;
      }
    }
  }
  float4 vals[ROWQ];
#pragma unroll
  for (int k = 0; k < ROWQ; ++k) {
    const int q = threadIdx.x + k * blockDim.x;
    vals[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q < nq) {
      const h16* bb = a.bias[e] + q * 4;
      float4 xn;
      xn.x = xv[k].x + (acc[k].x + (float)bb[0]);
      xn.y = xv[k].y + (acc[k].y + (float)bb[1]);
      xn.z = xv[k].z + (acc[k].z + (float)bb[2]);
      xn.w = xv[k].w + (acc[k].w + (float)bb[3]);
      *(float4*)(xr + q * 4) = xn;
      vals[k] = r16x4(xn);
    }
  }
  ln_row4(vals, d, a.g[e], a.b[e], a.a[e] + (size_t)r * d, red);
}

// ROWS: one workgroup per z row r.
//   init  : z[r] = init_latents(ctx)[r] (delta mode, fp16 arithmetic)
//   euler : v = fp16(sum_kc Pout[kc][i] + b_out) for the chunk c, row i owning z row r;
//           z[r] = fp16(z[r] + fp16(dt v))   (z_out[r] = z[r] after the last step)
// then, unless this was the last step, the next step's rows: for every expert c2 that reads z row
// r: x = fp16(fp16(z + pos[r]) + [current rows] tau), residual x = that, a = LN_self of block 0.
struct RowsArgs {
  const h16* ctx;
  float* ctx_mom;      // init: [C][2] (mean, rstd) of the fp16 context rows
  float* z;
  h16* z_out;
  const float* Pout[4];
  const h16* bout[4];
  float* x[4];
  const h16* pos[4];
  const h16* tau[4];
  const h16* g[4];
  const h16* b[4];
  h16* a[4];
  float dt;
  int euler, last, ks, d, C, CS, nch;
};

__global__ void __launch_bounds__(ROWT) k_rows(RowsArgs a) {
  __shared__ float red[ROWT / 64];
  const int r = blockIdx.x, d = a.d, nq = d / 4;
  float4 zv[ROWQ];
  if (!a.euler) {
    // moments of context rows r, r + gridDim.x, ... (read by the cross K/V GEMV)
    for (int cr = r; cr < a.C; cr += gridDim.x) {
      const h16* row = a.ctx + (size_t)cr * d;
      float sm = 0.f;
      for (int c = threadIdx.x; c < d; c += blockDim.x) sm += (float)row[c];
      const float mu = block_sum(sm, red) / (float)d;
      float sq = 0.f;
      for (int c = threadIdx.x; c < d; c += blockDim.x) {
        const float t = (float)row[c] - mu;
        sq += t * t;
      }
      const float rs = 1.0f / sqrtf(block_sum(sq, red) / (float)d + LN_EPS);
      if (threadIdx.x == 0) {
        a.ctx_mom[2 * cr] = mu;
        a.ctx_mom[2 * cr + 1] = rs;
      }
    }
    const h16* last = a.ctx + (size_t)(a.C - 1) * d;
    const h16* prev = a.ctx + (size_t)(a.C - 2) * d;
    const float step = (float)(r + 1);
#pragma unroll
    for (int k = 0; k < ROWQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      zv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (q < nq) {
        float o[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float lv = (float)last[q * 4 + t];
          const float delta = r16(lv - (float)prev[q * 4 + t]);
          o[t] = r16(lv + r16(step * delta));
        }
        zv[k] = make_float4(o[0], o[1], o[2], o[3]);
        *(float4*)(a.z + (size_t)r * d + q * 4) = zv[k];
      }
    }
  } else {
    const int c = r / a.CS, i = r - c * a.CS;
    const size_t pst = (size_t)a.CS * d;
    const float* Pr = a.Pout[c] + (size_t)i * d;
    float4 acc[ROWQ], zo[ROWQ];
#pragma unroll
    for (int k = 0; k < ROWQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      if (q < nq) {
        acc[k] = *(const float4*)(Pr + q * 4);
        zo[k] = *(const float4*)(a.z + (size_t)r * d + q * 4);
      }
    }
    for (int kc = 1; kc < a.ks; ++kc) {
#pragma unroll
      for (int k = 0; k < ROWQ; ++k) {
        const int q = threadIdx.x + k * blockDim.x;
        if (q < nq) {
          const float4 t = *(const float4*)(Pr + kc * pst + q * 4);
          acc[k].x += t.x; acc[k].y += t.y; acc[k].z += t.z; acc[k].w += t.w;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < ROWQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      zv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (q < nq) {
        const h16* bo = a.bout[c] + q * 4;
        float4 zn;
        zn.x = r16(zo[k].x + r16(a.dt * r16(acc[k].x + (float)bo[0])));
        zn.y = r16(zo[k].y + r16(a.dt * r16(acc[k].y + (float)bo[1])));
        zn.z = r16(zo[k].z + r16(a.dt * r16(acc[k].z + (float)bo[2])));
        zn.w = r16(zo[k].w + r16(a.dt * r16(acc[k].w + (float)bo[3])));
        *(float4*)(a.z + (size_t)r * d + q * 4) = zn;
        if (a.last) {
          h16* zo16 = a.z_out + (size_t)r * d + q * 4;
          zo16[0] = (h16)zn.x; zo16[1] = (h16)zn.y; zo16[2] = (h16)zn.z; zo16[3] = (h16)zn.w;
        }
        zv[k] = zn;
      }
    }
  }
  if (a.last) return;
  for (int c2 = 0; c2 < a.nch; ++c2) {
    if (r >= (c2 + 1) * a.CS) continue;          // expert c2 reads z rows [0, (c2+1)*CS)
    const bool cur = r >= c2 * a.CS;
    float4 vals[ROWQ];
#pragma unroll
    for (int k = 0; k < ROWQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      vals[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (q < nq) {
        const h16* pp = a.pos[c2] + (size_t)r * d + q * 4;
        const h16* tt = a.tau[c2] + q * 4;
        float o[4] = {zv[k].x, zv[k].y, zv[k].z, zv[k].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float xv = r16(o[t] + (float)pp[t]);
          if (cur) xv = r16(xv + (float)tt[t]);
          o[t] = xv;
        }
        vals[k] = make_float4(o[0], o[1], o[2], o[3]);
        *(float4*)(a.x[c2] + (size_t)r * d + q * 4) = vals[k];
      }
    }
    ln_row4(vals, d, a.g[c2], a.b[c2], a.a[c2] + (size_t)r * d, red);
  }
}

// ---------------------------------------------------------------------------- host side
struct Plan {
  int d, fd, CS, E, NL, C, KD, H, nch;
  int ks_qkv, ks_o, ks_w1, ks_w2, ks_out, ks_kv, ks_tau;
};

Plan make_plan(const cfh_flow_dims* dm) {
  Plan p;
  p.d = dm->d; p.fd = dm->ffn_mult * dm->d; p.CS = dm->chunk_size; p.E = dm->flow_steps;
  p.NL = dm->layers; p.C = dm->ctx_rows; p.KD = dm->draft_length; p.H = dm->heads;
  p.nch = p.KD / p.CS;
  p.ks_qkv = ksplit_for(p.nch, 3 * p.d / 16, p.d, p.KD);
  p.ks_o = ksplit_for(p.nch, p.d / 16, p.d, p.KD);
  p.ks_w1 = ksplit_for(p.nch, p.fd / 16, p.d, p.KD);
  p.ks_w2 = ksplit_for(p.nch, p.d / 16, p.fd, p.KD);
  p.ks_out = ksplit_for(p.nch, p.d / 16, p.d, p.CS);
  p.ks_kv = ksplit_for(p.nch * p.NL, 2 * p.d / 16, p.d, p.C);
  p.ks_tau = ksplit_for(p.nch, p.d / 16, p.d, p.E);
  return p;
}

struct WS {
  float* z;
  float* x[4];
  h16* abuf[4];
  h16* attn[4];
  h16* g[4];
  float* P[4];        // partials of the current GEMV
  float* Pw1[4];      // W1 partials (read by GELU)
  h16* tau[4];        // [E][d]
  h16* kvc[4];        // [L][2][C][d]
  float* Pkv;         // [nch][L][ks][C][2d]
  float* Ptau;        // [nch][ks][E][d]
  float* ctx_mom;     // [C][2]
  size_t total;
};

WS carve(const Plan& p, char* base) {
  WS w = {};
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* q = base ? base + off : nullptr;
    off = cfh::align256(off + bytes);
    return q;
  };
  const size_t d = p.d, fd = p.fd;
  w.z = (float*)take((size_t)p.KD * d * 4);
  for (int c = 0; c < p.nch; ++c) {
    const size_t S = (size_t)(c + 1) * p.CS;
    w.x[c] = (float*)take(S * d * 4);
    w.abuf[c] = (h16*)take(S * d * 2);
    w.attn[c] = (h16*)take(S * d * 2);
    w.g[c] = (h16*)take(S * fd * 2);
    size_t pmax = (size_t)p.ks_qkv * S * 3 * d;
    pmax = std::max(pmax, (size_t)p.ks_o * S * d);
    pmax = std::max(pmax, (size_t)p.ks_w2 * S * d);
    pmax = std::max(pmax, (size_t)p.ks_out * p.CS * d);
    w.P[c] = (float*)take(pmax * 4);
    w.Pw1[c] = (float*)take((size_t)p.ks_w1 * S * fd * 4);
    w.tau[c] = (h16*)take((size_t)p.E * d * 2);
    w.kvc[c] = (h16*)take((size_t)p.NL * 2 * p.C * d * 2);
  }
  w.Pkv = (float*)take((size_t)p.nch * p.NL * p.ks_kv * p.C * 2 * d * 4);
  w.Ptau = (float*)take((size_t)p.nch * p.ks_tau * p.E * d * 4);
  w.ctx_mom = (float*)take((size_t)p.C * 2 * 4);
  w.total = off;
  return w;
}

int launch_attn(const AttnArgs& a, int nex, int sq_max, int sk_max, hipStream_t st) {
  const size_t lds = (size_t)(sq_max + 2 * sk_max) * a.hd * 2;
  if (lds > 120 * 1024 || sq_max > MAXR || sk_max > MAXR) return CFH_E_UNSUPPORTED;
  hipLaunchKernelGGL(k_attn, dim3(nex * a.heads), dim3(1024), lds, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}


// One launch of one chunk expert's Euler step.  Kernel k of block l (k = 0..11):
//   0 QKV, 1 self attention, 2 O, 3 NORM(LN_cross), 4 QC, 5 cross attention, 6 OC, 7 NORM(LN_ffn),
//   8 W1, 9 GELU, 10 W2, 11 NORM(next LN);  l == NL, k == 0: out_proj on the current chunk rows.
constexpr int KPB = 12;   // kernels per block and expert

int expert_kernel(const Plan& p, const cfh::ExpertLayout& L, const WS& w, const void* expert, int c, int l,
                  int k, hipStream_t st) {
  const int d = p.d, fd = p.fd, CS = p.CS, NL = p.NL, C = p.C, H = p.H;
  const int S = (c + 1) * CS;
  auto PTR = [&](size_t off) { return (const char*)expert + off; };
  auto BLK = [&](int ll) { return L.blk0 + (size_t)ll * L.blkstride; };
  if (l == NL) {
    GemvArgs a = {};
    a.nex = 1; a.nl = 1; a.E = p.E; a.ks = p.ks_out; a.tiles = d / 16; a.N = d; a.K = d;
    GemvEx& x = a.ex[0];
    x.w = (const h16x8*)PTR(L.out);
    x.a = w.abuf[c] + (size_t)c * CS * d;   // out_norm rows of the current chunk
    x.lda = d; x.pout = w.P[c]; x.rows = CS;
    return launch_gemv<SRC_BUF>(a, CS, st);
  }
  const size_t B = BLK(l);
  GemvArgs a = {};
  a.nex = 1; a.nl = 1; a.E = p.E;
  GemvEx& x = a.ex[0];
  x.lda = d; x.pout = w.P[c]; x.rows = S;
  AttnArgs at = {};
  at.d = d; at.heads = H; at.hd = d / H; at.P[0] = w.P[c]; at.out[0] = w.attn[c]; at.Sq[0] = S;
  NormArgs nm = {};
  nm.nex = 1; nm.d = d; nm.x[0] = w.x[c]; nm.P[0] = w.P[c]; nm.a[0] = w.abuf[c]; nm.rows[0] = S;
  switch (k) {
    case 0:  // QKV
      a.ks = p.ks_qkv; a.tiles = 3 * d / 16; a.N = 3 * d; a.K = d;
      x.w = (const h16x8*)PTR(B + L.qkv); x.a = w.abuf[c];
      return launch_gemv<SRC_BUF>(a, S, st);
    case 1:  // causal self attention
      at.ks = p.ks_qkv; at.ldp = 3 * d; at.causal = 1; at.bias[0] = (const h16*)PTR(B + L.qkv_b);
      at.kv[0] = nullptr; at.Sk[0] = S;
      return launch_attn(at, 1, S, S, st);
    case 2:  // O
      a.ks = p.ks_o; a.tiles = d / 16; a.N = d; a.K = d;
      x.w = (const h16x8*)PTR(B + L.o); x.a = w.attn[c];
      return launch_gemv<SRC_BUF>(a, S, st);
    case 3:  // residual + LN_cross
      nm.ks = p.ks_o; nm.bias[0] = (const h16*)PTR(B + L.o_b);
      nm.g[0] = (const h16*)PTR(B + L.xn_w); nm.b[0] = (const h16*)PTR(B + L.xn_b);
      hipLaunchKernelGGL(k_norm, dim3(S), dim3(ROWT), 0, st, nm);
      CFH_LAUNCH_CHECK();
      return CFH_OK;
    case 4:  // QC
      a.ks = p.ks_o; a.tiles = d / 16; a.N = d; a.K = d;
      x.w = (const h16x8*)PTR(B + L.qc); x.a = w.abuf[c];
      return launch_gemv<SRC_BUF>(a, S, st);
    case 5:  // cross attention over the hoisted context K/V
      at.ks = p.ks_o; at.ldp = d; at.causal = 0; at.bias[0] = (const h16*)PTR(B + L.qc_b);
      at.kv[0] = w.kvc[c] + (size_t)l * 2 * C * d; at.Sk[0] = C;
      return launch_attn(at, 1, S, C, st);
    case 6:  // OC
      a.ks = p.ks_o; a.tiles = d / 16; a.N = d; a.K = d;
      x.w = (const h16x8*)PTR(B + L.oc); x.a = w.attn[c];
      return launch_gemv<SRC_BUF>(a, S, st);
    case 7:  // residual + LN_ffn
      nm.ks = p.ks_o; nm.bias[0] = (const h16*)PTR(B + L.oc_b);
      nm.g[0] = (const h16*)PTR(B + L.fn_w); nm.b[0] = (const h16*)PTR(B + L.fn_b);
      hipLaunchKernelGGL(k_norm, dim3(S), dim3(ROWT), 0, st, nm);
      CFH_LAUNCH_CHECK();
      return CFH_OK;
    case 8:  // W1
      a.ks = p.ks_w1; a.tiles = fd / 16; a.N = fd; a.K = d;
      x.w = (const h16x8*)PTR(B + L.w1); x.a = w.abuf[c]; x.pout = w.Pw1[c];
      return launch_gemv<SRC_BUF>(a, S, st);
    case 9: {  // GELU
      GeluArgs ge = {};
      ge.nex = 1; ge.ks = p.ks_w1; ge.N = fd;
      ge.P[0] = w.Pw1[c]; ge.b[0] = (const h16*)PTR(B + L.w1_b); ge.g[0] = w.g[c]; ge.rows[0] = S;
      hipLaunchKernelGGL(k_gelu, dim3(192), dim3(256), 0, st, ge);
      CFH_LAUNCH_CHECK();
      return CFH_OK;
    }
    case 10:  // W2
      a.ks = p.ks_w2; a.tiles = d / 16; a.N = d; a.K = fd;
      x.w = (const h16x8*)PTR(B + L.w2); x.a = w.g[c]; x.lda = fd;
      return launch_gemv<SRC_BUF>(a, S, st);
    case 11:  // residual + LayerNorm of the next block (out_norm after the last block)
      nm.ks = p.ks_w2; nm.bias[0] = (const h16*)PTR(B + L.w2_b);
      if (l + 1 < NL) {
        nm.g[0] = (const h16*)PTR(BLK(l + 1) + L.sn_w); nm.b[0] = (const h16*)PTR(BLK(l + 1) + L.sn_b);
      } else {
        nm.g[0] = (const h16*)PTR(L.on_w); nm.b[0] = (const h16*)PTR(L.on_b);
      }
      hipLaunchKernelGGL(k_norm, dim3(S), dim3(ROWT), 0, st, nm);
      CFH_LAUNCH_CHECK();
      return CFH_OK;
  }
  return CFH_E_INVALID;
}

// Side streams and fork/join events (one set per device, created on first use).
struct SideStreams {
  hipStream_t st[4];
  hipEvent_t fork;
  hipEvent_t join[4];
};

SideStreams* side_streams(int* status) {
  static SideStreams cache[64];
  static bool made[64];
  static std::mutex mu;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) {
    *status = cfh::set_hip_error(e == hipSuccess ? hipErrorInvalidDevice : e);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  SideStreams& s = cache[dev];
  if (!made[dev]) {
    s.st[0] = nullptr;
    for (int c = 1; c < 4; ++c)
      if ((e = hipStreamCreateWithFlags(&s.st[c], hipStreamNonBlocking)) != hipSuccess) break;
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s.fork, hipEventDisableTiming);
    for (int c = 0; c < 4 && e == hipSuccess; ++c) e = hipEventCreateWithFlags(&s.join[c], hipEventDisableTiming);
    if (e != hipSuccess) {
      *status = cfh::set_hip_error(e);
      return nullptr;
    }
    made[dev] = true;
  }
  *status = CFH_OK;
  return &s;
}

}  // namespace

extern "C" {

int cfh_caps(const cfh_flow_dims* dims, int batch, int64_t* ws_bytes) {
  if (!cfh::flow_dims_ok(dims) || batch < 1) return CFH_E_UNSUPPORTED;
  if (dims->d > ROWT * ROWE) return CFH_E_UNSUPPORTED;
  const Plan p = make_plan(dims);
  const WS w = carve(p, nullptr);
  if (ws_bytes) *ws_bytes = (int64_t)w.total;
  return CFH_OK;
}

int cfh_flow_integrate(const cfh_flow_dims* dm, const void* const* experts, const void* ctx, void* z_out,
                       void* ws_ptr, int batch, void* stream) {
  if (!cfh::flow_dims_ok(dm) || dm->d > ROWT * ROWE) return CFH_E_UNSUPPORTED;
  if (!experts || !ctx || !z_out || !ws_ptr || batch < 1) return CFH_E_INVALID;
  const Plan p = make_plan(dm);
  for (int c = 0; c < p.nch; ++c)
    if (!experts[c]) return CFH_E_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const cfh::ExpertLayout L = cfh::expert_layout(dm);
  const WS w = carve(p, (char*)ws_ptr);
  const int d = p.d, CS = p.CS, E = p.E, NL = p.NL, C = p.C, KD = p.KD, nch = p.nch;
  int rc = CFH_OK;
  SideStreams* side = nullptr;
  if (nch > 1 && !(side = side_streams(&rc))) return rc;
  auto PTR = [&](int c, size_t off) { return (const char*)experts[c] + off; };
  auto BLK = [&](int l) { return L.blk0 + (size_t)l * L.blkstride; };

  for (int b = 0; b < batch; ++b) {
    const h16* ctx_b = (const h16*)ctx + (size_t)b * C * d;
    h16* zo_b = (h16*)z_out + (size_t)b * KD * d;

    // ---- per draft: time embeddings of every step, z0 + step-0 rows, cross K/V of every block
    {
      GemvArgs a = {};
      a.nex = nch; a.nl = 1; a.ks = p.ks_tau; a.tiles = d / 16; a.N = d; a.K = d; a.E = E;
      for (int c = 0; c < nch; ++c) {
        GemvEx& x = a.ex[c];
        x.w = (const h16x8*)PTR(c, L.tw2);
        x.g0 = (const h16*)PTR(c, L.tw0);
        x.b0 = (const h16*)PTR(c, L.tb0);
        x.pout = w.Ptau + (size_t)c * p.ks_tau * E * d;
        x.rows = E;
      }
      if ((rc = launch_gemv<SRC_TAU>(a, E, st))) return rc;
      ReduceArgs r = {};
      r.nex = nch; r.nl = 1; r.ks = p.ks_tau; r.rows = E; r.N = d; r.d = d; r.kv = 0;
      for (int c = 0; c < nch; ++c) {
        r.P[c] = a.ex[c].pout;
        r.b[c] = (const h16*)PTR(c, L.tb2);
        r.out[c] = w.tau[c];
      }
      hipLaunchKernelGGL(k_reduce, dim3(256), dim3(256), 0, st, r);
      CFH_LAUNCH_CHECK();
    }
    // ---- z0 and the step-0 rows
    {
      RowsArgs r = {};
      r.ctx = ctx_b; r.ctx_mom = w.ctx_mom; r.z = w.z; r.z_out = zo_b; r.euler = 0; r.last = 0; r.d = d; r.C = C; r.CS = CS;
      r.nch = nch;
      for (int c = 0; c < nch; ++c) {
        r.x[c] = w.x[c]; r.pos[c] = (const h16*)PTR(c, L.pos); r.tau[c] = w.tau[c];
        r.g[c] = (const h16*)PTR(c, BLK(0) + L.sn_w); r.b[c] = (const h16*)PTR(c, BLK(0) + L.sn_b);
        r.a[c] = w.abuf[c];
      }
      hipLaunchKernelGGL(k_rows, dim3(KD), dim3(ROWT), 0, st, r);
      CFH_LAUNCH_CHECK();
    }

    {
      GemvArgs a = {};
      a.nex = nch; a.nl = NL; a.ks = p.ks_kv; a.tiles = 2 * d / 16; a.N = 2 * d; a.K = d; a.E = E;
      a.wstride = (long long)L.blkstride; a.vstride = (long long)L.blkstride;
      for (int c = 0; c < nch; ++c) {
        GemvEx& x = a.ex[c];
        x.w = (const h16x8*)PTR(c, BLK(0) + L.kv);
        x.a = ctx_b;
        x.g0 = (const h16*)PTR(c, BLK(0) + L.cn_w);
        x.b0 = (const h16*)PTR(c, BLK(0) + L.cn_b);
        x.pout = w.Pkv + (size_t)c * NL * p.ks_kv * C * 2 * d;
        x.mom = w.ctx_mom;
        x.rows = C;
      }
      if ((rc = launch_gemv<SRC_CTX>(a, C, st))) return rc;
      ReduceArgs r = {};
      r.nex = nch; r.nl = NL; r.ks = p.ks_kv; r.rows = C; r.N = 2 * d; r.d = d; r.kv = 1;
      r.vstride = (long long)L.blkstride;
      for (int c = 0; c < nch; ++c) {
        r.P[c] = a.ex[c].pout;
        r.b[c] = (const h16*)PTR(c, BLK(0) + L.kv_b);
        r.out[c] = w.kvc[c];
      }
      hipLaunchKernelGGL(k_reduce, dim3(1024), dim3(256), 0, st, r);
      CFH_LAUNCH_CHECK();
    }
    for (int s = 0; s < E; ++s) {
      // The chunk experts are independent within an Euler step (their inputs are slices of the
      // step's z): expert 0 runs on the caller's stream, the others on side streams, so one
      // expert's boundary kernels overlap the other's weight streaming.  Join before the update.
      if (nch > 1) {
        CFH_HIP(hipEventRecord(side->fork, st));
        for (int c = 1; c < nch; ++c) CFH_HIP(hipStreamWaitEvent(side->st[c], side->fork, 0));
      }
      // Launches alternate between the experts' streams, kernel by kernel.
      for (int l = 0; l <= NL; ++l) {
        const int nk = l < NL ? KPB : 1;
        for (int k = 0; k < nk; ++k)
          for (int c = 0; c < nch; ++c)
            if ((rc = expert_kernel(p, L, w, experts[c], c, l, k, c == 0 ? st : side->st[c]))) return rc;
      }
      if (nch > 1) {
        for (int c = 1; c < nch; ++c) {
          CFH_HIP(hipEventRecord(side->join[c], side->st[c]));
          CFH_HIP(hipStreamWaitEvent(st, side->join[c], 0));
        }
      }
      RowsArgs r = {};
      r.ctx = ctx_b; r.z = w.z; r.z_out = zo_b; r.euler = 1; r.last = (s + 1 == E); r.ks = p.ks_out;
      r.dt = 1.0f / (float)E; r.d = d; r.C = C; r.CS = CS; r.nch = nch;
      for (int c = 0; c < nch; ++c) {
        r.Pout[c] = w.P[c]; r.bout[c] = (const h16*)PTR(c, L.out_b);
        r.x[c] = w.x[c]; r.pos[c] = (const h16*)PTR(c, L.pos);
        r.tau[c] = w.tau[c] + (size_t)(s + 1 < E ? s + 1 : s) * d;
        r.g[c] = (const h16*)PTR(c, BLK(0) + L.sn_w); r.b[c] = (const h16*)PTR(c, BLK(0) + L.sn_b);
        r.a[c] = w.abuf[c];
      }
      hipLaunchKernelGGL(k_rows, dim3(KD), dim3(ROWT), 0, st, r);
      CFH_LAUNCH_CHECK();
    }
  }
  return CFH_OK;
}

}  // extern "C"
