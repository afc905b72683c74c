// The chain-flow velocity net + Euler integrator on MI355X: TreeFlowDrafter.predict_hidden.
//
// Reference semantics (cf/ = src/chain_flow/): init_latents cf/drafters/tree_flow.py:150-161,
// integrate :229-235, flow_velocity/_chunk_args :163-190, HiddenKVFlowExpert.pre_blocks /
// post_blocks cf/drafters/chunked_flow.py:333-384, HiddenKVFlowBlock.forward :185-202; fused-kernel
// numerics cf/csrc/fused_block.cu:280-325, 452-668, 674-722 (fp32 residual, fp16-parked LayerNorm
// rows, fp16 q/k/v, attention and GELU outputs, cross K/V hoisted once per draft).
//
// Execution plan (one launch sequence per draft, every launch on the caller's stream):
//   init  : z0 = init_latents(ctx); x rows of step 0 (pre_blocks) and their LayerNorm moments
//   kv    : cross-attention K/V of every block of every chunk expert (once per draft)
//   tau   : time_mlp(tau_s) for all E steps (tau only depends on s)
//   per Euler step s, per block l, both chunk experts in the same launch:
//     QKV : LN_self(x) -> q,k,v (fp16); the last wave to finish a head runs its causal attention
//     O   : x += attn W_o^T + b_o                          (+ LayerNorm moments of the new x)
//     QC  : LN_cross(x) -> q (fp16); the last wave of a head runs cross attention on the hoisted K/V
//     OC  : x += attn W_oc^T + b_oc                        (+ moments)
//     W1  : g = GELU(LN_ffn(x) W1^T + b1) (fp16)
//     W2  : x += g W2^T + b2                               (+ moments)
//   OUT   : v = out_proj(out_norm(x[cur rows])); z = fp16(z + dt v); next step's pre_blocks rows
//
// Every GEMV is a weight-streaming MFMA loop (cfh_common.h stream_tile): a wave owns one
// (n-tile of 16 outputs, k-chunk) unit and streams its contiguous packed fragments while the
// activation rows (<= 16) sit in LDS.  Split-K units leave fp32 partials; the last unit of a tile
// to finish (agent-scope counter) sums them in k-chunk order and runs the epilogue, so results do
// not depend on arrival order.  LayerNorm moments (sum, sum of squares of the fp16-parked row) are
// accumulated by the residual epilogues with fp32 atomics, so the next LayerNorm needs no extra
// pass over the row.
#include <stdio.h>

#include <algorithm>

#include "cfh_common.h"
#include "cfh_host.h"

namespace {

constexpr int WPB = 4;          // waves per workgroup
constexpr int PF = 8;           // fragment loads in flight per wave
constexpr int MAXR = 16;        // max activation rows per expert
constexpr float LN_EPS = 1e-5f;
constexpr int MAX_UNITS = 16384;  // split-K (tile, k-chunk) units per expert per phase

enum Kind { K_QKV = 0, K_O, K_QC, K_OC, K_W1, K_W2, K_OUT, K_KV, K_TAU };

struct PhaseEx {
  const h16x8* w;        // packed matrix of this phase (layer 0 of the unit range for KV)
  const h16* bias;       // [N]
  const h16* lng;        // LayerNorm gamma (A1/KV) | time_mlp.0.weight (TAU)
  const h16* lnb;        // LayerNorm beta          | time_mlp.0.bias   (TAU)
  const float* st_in;    // [MAXR][2] LayerNorm moments of x (A1)
  float* st_out;         // [MAXR][2] moments of the updated x (residual epilogues)
  float* x;              // [srows][d] fp32 residual
  h16* x16;              // [srows][d] fp16 copy of x (what LayerNorm reads)
  h16* qkv;              // [srows][3d]
  h16* attn;             // [srows][d]
  h16* g;                // [srows][f*d]
  const h16* kv;         // [2][C][d] cross K/V of this block (QC)
  h16* out;              // KV: [L][2][C][d]   TAU: [E][d]
  const h16* pos;        // OUT: position_embedding [KD][d]
  const h16* tau_next;   // OUT: time_mlp(tau_{s+1}) [d]
  float* st_next;        // OUT: [MAXR][2] moments of next step's x
  float* x_next;         // OUT: next step's residual rows (the other ping-pong buffer)
  h16* x16_next;         // OUT: fp16 copy of x_next
  int rows;              // activation rows of this phase
  int row0;              // first x row read by this phase (OUT: current chunk)
  int srows;             // rows of this expert's sequence (prev + current)
};

struct PhaseArgs {
  PhaseEx ex[4];
  int nex, nl;
  long long wstride, vstride;   // KV: bytes between consecutive layers' packed / vector params
  int d, N, K, ksplit, tiles, heads, hd, CS, C, E, FD;
  float dt;
  int has_next;
  float* z;                     // [KD][d] fp32 (fp16-valued)
  h16* z_out;                   // [KD][d] fp16 (last step)
  float* partials;              // [units][256]
  unsigned* tile_ctr;           // [nex * nl * tiles]
  unsigned* head_ctr;           // [nex * heads]
  const h16* ctx;               // [C][d]
};

// ---------------------------------------------------------------------------- attention
// One wave computes softmax(q k^T / sqrt(hd) [+ causal]) v for one head: rows Sq queries, Sk keys.
// Lane owns head dims [lane*dpl, lane*dpl + dpl).  Scores are reduced across the wave.
__device__ void wave_attention(const h16* q, int ldq, const h16* k, int ldk, const h16* v, int ldv,
                               int Sq, int Sk, bool causal, int hd, h16* out, int ldo) {
  const int lane = threadIdx.x & 63;
  const int dpl = hd / 64;
  const int c0 = lane * dpl;
  const float scale = 1.0f / sqrtf((float)hd);
  for (int i = 0; i < Sq; ++i) {
    const int nk = causal ? i + 1 : Sk;
    float sc[MAXR];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < MAXR; ++j) {
      sc[j] = -INFINITY;
      if (j < nk) {
        float p = 0.f;
        for (int t = 0; t < dpl; ++t) p += (float)q[i * ldq + c0 + t] * (float)k[j * ldk + c0 + t];
        const float s = wave_sum(p) * scale;
        sc[j] = s;
        m = fmaxf(m, s);
      }
    }
    float den = 0.f;
#pragma unroll
    for (int j = 0; j < MAXR; ++j) {
      const float e = (j < nk) ? expf(sc[j] - m) : 0.f;
      sc[j] = e;
      den += e;
    }
    const float inv = 1.0f / den;
    for (int t = 0; t < dpl; ++t) {
      float o = 0.f;
#pragma unroll
      for (int j = 0; j < MAXR; ++j)
        if (j < nk) o += sc[j] * inv * (float)v[j * ldv + c0 + t];
      out[i * ldo + c0 + t] = (h16)o;
    }
  }
}

// ---------------------------------------------------------------------------- A staging
__device__ __forceinline__ void ln_moments(const float* st, int row, int d, float& mean, float& rstd) {
  const float s = st[row * 2], q = st[row * 2 + 1];
  mean = s / (float)d;
  const float var = fmaxf(q / (float)d - mean * mean, 0.f);
  rstd = 1.0f / sqrtf(var + LN_EPS);
}

template <int KIND>
__device__ void stage_A(const PhaseArgs& a, const PhaseEx& ep, int l, int kc, h16* As, int lda) {
  __shared__ float sm_mean[MAXR], sm_rstd[MAXR];
  const int KC = a.K / a.ksplit;
  const int k0 = kc * KC;
  const int rows = ep.rows;
  const int nvec = KC / 8;
  if constexpr (KIND == K_QKV || KIND == K_QC || KIND == K_W1 || KIND == K_OUT) {
    if (threadIdx.x < rows) {
      float mu, rs;
      ln_moments(ep.st_in, ep.row0 + threadIdx.x, a.d, mu, rs);
      sm_mean[threadIdx.x] = mu;
      sm_rstd[threadIdx.x] = rs;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < rows * nvec; idx += blockDim.x) {
      const int i = idx / nvec, kk = (idx - i * nvec) * 8;
      const h16x8 xv = *(const h16x8*)(ep.x16 + (size_t)(ep.row0 + i) * a.d + k0 + kk);
      const h16x8 gv = *(const h16x8*)(ep.lng + k0 + kk);
      const h16x8 bv = *(const h16x8*)(ep.lnb + k0 + kk);
      const float mu = sm_mean[i], rs = sm_rstd[i];
      h16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (h16)(((float)xv[e] - mu) * rs * (float)gv[e] + (float)bv[e]);
      *(h16x8*)(As + i * lda + kk) = o;
    }
  } else if constexpr (KIND == K_O || KIND == K_OC || KIND == K_W2) {
    const h16* src = (KIND == K_W2) ? ep.g : ep.attn;
    const int ld = (KIND == K_W2) ? a.FD : a.d;
    for (int idx = threadIdx.x; idx < rows * nvec; idx += blockDim.x) {
      const int i = idx / nvec, kk = (idx - i * nvec) * 8;
      *(h16x8*)(As + i * lda + kk) = *(const h16x8*)(src + (size_t)i * ld + k0 + kk);
    }
  } else if constexpr (KIND == K_KV) {
    // context_norm(ctx) of block l: moments of the fp16 context rows computed here (two-pass).
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int i = wave; i < rows; i += blockDim.x / 64) {
      const h16* cr = a.ctx + (size_t)i * a.d;
      float s = 0.f;
      for (int c = lane; c < a.d; c += 64) s += (float)cr[c];
      s = wave_sum(s);
      const float mu = s / (float)a.d;
      float q = 0.f;
      for (int c = lane; c < a.d; c += 64) {
        const float t = (float)cr[c] - mu;
        q += t * t;
      }
      q = wave_sum(q);
      if (lane == 0) {
        sm_mean[i] = mu;
        sm_rstd[i] = 1.0f / sqrtf(q / (float)a.d + LN_EPS);
      }
    }
    __syncthreads();
    const h16* gw = (const h16*)((const char*)ep.lng + (size_t)l * a.vstride);
    const h16* gb = (const h16*)((const char*)ep.lnb + (size_t)l * a.vstride);
    for (int idx = threadIdx.x; idx < rows * nvec; idx += blockDim.x) {
      const int i = idx / nvec, kk = (idx - i * nvec) * 8;
      const h16x8 xv = *(const h16x8*)(a.ctx + (size_t)i * a.d + k0 + kk);
      const h16x8 gv = *(const h16x8*)(gw + k0 + kk);
      const h16x8 bv = *(const h16x8*)(gb + k0 + kk);
      const float mu = sm_mean[i], rs = sm_rstd[i];
      h16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (h16)(((float)xv[e] - mu) * rs * (float)gv[e] + (float)bv[e]);
      *(h16x8*)(As + i * lda + kk) = o;
    }
  } else if constexpr (KIND == K_TAU) {
    // rows = Euler steps: a_s = fp16(silu(fp16(tau_s * w0 + b0))), tau_s = fp16(s / E)
    for (int idx = threadIdx.x; idx < rows * nvec; idx += blockDim.x) {
      const int i = idx / nvec, kk = (idx - i * nvec) * 8;
      const float tau = r16((float)i * (1.0f / (float)a.E));
      h16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float h = r16(tau * (float)ep.lng[k0 + kk + e] + (float)ep.lnb[k0 + kk + e]);
        o[e] = (h16)silu(h);
      }
      *(h16x8*)(As + i * lda + kk) = o;
    }
  }
  __syncthreads();
}

// Sum the 16 lanes of a 16-lane group (lanes sharing lane>>4).
__device__ __forceinline__ float group16_sum(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  return v;
}

// Residual update of one (row, col) value with LayerNorm-moment accumulation.
__device__ __forceinline__ void moments_add(float* st, int row, bool valid, float xv16) {
  float s1 = valid ? xv16 : 0.f, s2 = valid ? xv16 * xv16 : 0.f;
  s1 = group16_sum(s1);
  s2 = group16_sum(s2);
  if (valid && (threadIdx.x & 15) == 0) {
    atomicAdd(st + row * 2, s1);
    atomicAdd(st + row * 2 + 1, s2);
  }
}

// ---------------------------------------------------------------------------- phase kernel
template <int KIND>
__global__ void __launch_bounds__(WPB * 64) k_phase(PhaseArgs a) {
  extern __shared__ __align__(16) h16 As[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per_ex = a.nl * a.ksplit * a.tiles;
  const int u = blockIdx.x * WPB + wave;
  const int u0 = blockIdx.x * WPB;
  const int e = u0 / per_ex;
  int rem = u0 - e * per_ex;
  const int l = rem / (a.ksplit * a.tiles);
  rem -= l * a.ksplit * a.tiles;
  const int kc = rem / a.tiles;
  const int t = (u - u0) + (rem - kc * a.tiles);  // tile of this wave (WG never straddles (e,l,kc))
  const PhaseEx& ep = a.ex[e];
  const int KC = a.K / a.ksplit;
  const int lda = KC + 8;

  stage_A<KIND>(a, ep, l, kc, As, lda);

  const h16x8* wbase = (const h16x8*)((const char*)ep.w + (size_t)l * a.wstride);
  const h16x8* wp = wbase + packed_index(t, kc * (KC / 32), a.K, 0);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = stream_tile<PF>(wp, As, lda, ep.rows, KC / 32, acc);

  const int col = lane & 15;
  const int rbase = 4 * (lane >> 4);
  if (a.ksplit > 1) {
    const size_t tix = ((size_t)e * a.nl + l) * a.tiles + t;
    float* pp = a.partials + tix * a.ksplit * 256;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (rbase + j < ep.rows) pp[kc * 256 + (rbase + j) * 16 + col] = acc[j];
    const unsigned old = arrive_count(a.tile_ctr + tix);
    if (old != (unsigned)(a.ksplit - 1)) return;
    acquire_fence();
    reset_count(a.tile_ctr + tix);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float s = 0.f;
      if (rbase + j < ep.rows)
        for (int q = 0; q < a.ksplit; ++q) s += pp[q * 256 + (rbase + j) * 16 + col];
      acc[j] = s;
    }
  }

  const int n = t * 16 + col;
  const h16* bias = (const h16*)((const char*)ep.bias + (size_t)l * a.vstride);
  const float bn = (float)bias[n];
  if constexpr (KIND == K_QKV || KIND == K_QC) {
    const int ld = 3 * a.d;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (rbase + j < ep.rows) ep.qkv[(size_t)(rbase + j) * ld + n] = (h16)(acc[j] + bn);
    const int h = (n % a.d) / a.hd;
    const unsigned total = (KIND == K_QKV) ? 3u * (unsigned)(a.hd / 16) : (unsigned)(a.hd / 16);
    unsigned* hc = a.head_ctr + e * a.heads + h;
    const unsigned old = arrive_count(hc);
    if (old != total - 1) return;
    acquire_fence();
    reset_count(hc);
    const int c0 = h * a.hd;
    if constexpr (KIND == K_QKV) {
      wave_attention(ep.qkv + c0, ld, ep.qkv + a.d + c0, ld, ep.qkv + 2 * a.d + c0, ld, ep.rows, ep.rows,
                     true, a.hd, ep.attn + c0, a.d);
    } else {
      wave_attention(ep.qkv + c0, ld, ep.kv + c0, a.d, ep.kv + (size_t)a.C * a.d + c0, a.d, ep.rows, a.C,
                     false, a.hd, ep.attn + c0, a.d);
    }
  } else if constexpr (KIND == K_O || KIND == K_OC || KIND == K_W2) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = rbase + j;
      const bool valid = row < ep.rows;
      float x16v = 0.f;
      if (valid) {
        const size_t ix = (size_t)row * a.d + n;
        const float xn = ep.x[ix] + (acc[j] + bn);
        ep.x[ix] = xn;
        x16v = r16(xn);
        ep.x16[ix] = (h16)x16v;
      }
      moments_add(ep.st_out, row, valid, x16v);
    }
  } else if constexpr (KIND == K_W1) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (rbase + j < ep.rows) ep.g[(size_t)(rbase + j) * a.FD + n] = (h16)gelu_erf(acc[j] + bn);
  } else if constexpr (KIND == K_KV) {
    // output n < d -> K, else V; layout [L][2][C][d]
    const int part = n / a.d, nn = n - part * a.d;
    h16* o = ep.out + (((size_t)l * 2 + part) * a.C) * a.d;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (rbase + j < ep.rows) o[(size_t)(rbase + j) * a.d + nn] = (h16)(acc[j] + bn);
  } else if constexpr (KIND == K_TAU) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (rbase + j < ep.rows) ep.out[(size_t)(rbase + j) * a.d + n] = (h16)(acc[j] + bn);
  } else if constexpr (KIND == K_OUT) {
    // v = fp16(out_proj(out_norm(x_cur))); z = fp16(z + fp16(dt v)); then the next step's
    // pre_blocks rows fed by this z row: fp16(fp16(z + pos[row]) + [current rows] tau_next).
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = rbase + j;
      const bool valid = i < ep.rows;
      const int zr = e * a.CS + i;
      float zn = 0.f;
      if (valid) {
        const float v16 = r16(acc[j] + bn);
        zn = r16(a.z[(size_t)zr * a.d + n] + r16(a.dt * v16));
        a.z[(size_t)zr * a.d + n] = zn;
        if (!a.has_next) a.z_out[(size_t)zr * a.d + n] = (h16)zn;
      }
      if (a.has_next) {
        for (int c2 = 0; c2 < a.nex; ++c2) {
          const PhaseEx& e2 = a.ex[c2];
          const bool use = valid && zr < e2.srows;
          float xv = 0.f;
          if (use) {
            xv = r16(zn + (float)e2.pos[(size_t)zr * a.d + n]);
            if (zr >= c2 * a.CS) xv = r16(xv + (float)e2.tau_next[n]);
            e2.x_next[(size_t)zr * a.d + n] = xv;
            e2.x16_next[(size_t)zr * a.d + n] = (h16)xv;
          }
          // moments: every lane of the wave takes part in the shuffles
          float s1 = use ? xv : 0.f, s2 = use ? xv * xv : 0.f;
          s1 = group16_sum(s1);
          s2 = group16_sum(s2);
          if (use && (lane & 15) == 0) {
            atomicAdd(e2.st_next + zr * 2, s1);
            atomicAdd(e2.st_next + zr * 2 + 1, s2);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------- init kernel
// One workgroup per z row r: z0[r] = init_latents(ctx) (delta mode, fp16 arithmetic as in the
// expert dtype), then the step-0 pre_blocks rows of every expert that reads z row r, with their
// full-row LayerNorm moments.  Workgroups also clear the counters and the moment buffers of all
// later generations.
struct InitArgs {
  const h16* ctx;     // [C][d]
  float* z;           // [KD][d]
  int d, C, KD, CS, nch, init_mode;
  float* x[4];
  h16* x16[4];
  float* st0[4];      // generation-0 moments per expert [MAXR][2]
  const h16* pos[4];
  const h16* tau0[4]; // time_mlp(tau_0) per expert
  int srows[4];
  float* zero_f; size_t nzero_f;      // later-generation moments
  unsigned* zero_u; size_t nzero_u;   // counters
};

__global__ void __launch_bounds__(256) k_flow_init(InitArgs a) {
  const int r = blockIdx.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.nzero_f; i += (size_t)gridDim.x * blockDim.x)
    a.zero_f[i] = 0.f;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.nzero_u; i += (size_t)gridDim.x * blockDim.x)
    a.zero_u[i] = 0u;
  __shared__ float red[2][4][8];
  const h16* last = a.ctx + (size_t)(a.C - 1) * a.d;
  const h16* prev = a.ctx + (size_t)(a.C - 2) * a.d;
  const float step = (float)(r + 1);
  float s1[4] = {0, 0, 0, 0}, s2[4] = {0, 0, 0, 0};
  for (int c = threadIdx.x; c < a.d; c += blockDim.x) {
    const float lv = (float)last[c];
    float z0;
    if (a.init_mode == 1) {
      z0 = lv;  // repeat_last
    } else {
      const float delta = r16(lv - (float)prev[c]);
      z0 = r16(lv + r16(step * delta));
    }
    a.z[(size_t)r * a.d + c] = z0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (e >= a.nch || r >= a.srows[e]) continue;
      float xv = r16(z0 + (float)a.pos[e][(size_t)r * a.d + c]);
      if (r >= e * a.CS) xv = r16(xv + (float)a.tau0[e][c]);
      a.x[e][(size_t)r * a.d + c] = xv;
      a.x16[e][(size_t)r * a.d + c] = (h16)xv;
      s1[e] += xv;
      s2[e] += xv * xv;
    }
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float t1 = wave_sum(s1[e]), t2 = wave_sum(s2[e]);
    if (lane == 0) {
      red[0][e][wave] = t1;
      red[1][e][wave] = t2;
    }
  }
  __syncthreads();
  if (threadIdx.x < a.nch) {
    const int e = threadIdx.x;
    if (r < a.srows[e]) {
      float t1 = 0.f, t2 = 0.f;
      for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
        t1 += red[0][e][w];
        t2 += red[1][e][w];
      }
      a.st0[e][r * 2] = t1;
      a.st0[e][r * 2 + 1] = t2;
    }
  }
}

// ---------------------------------------------------------------------------- host side
struct WS {
  float* z;
  float* x[4][2];
  h16* x16[4][2];
  h16* qkv[4];
  h16* attn[4];
  h16* g[4];
  h16* tau[4];
  h16* kvc[4];
  float* stats;      // [ngen][nch][MAXR][2]
  float* partials;
  unsigned* tile_ctr;
  unsigned* head_ctr;
  size_t total, ngen, stats_floats, n_tile_ctr, n_head_ctr, partial_floats;
};

int ksplit_for(int nex_units, int tiles, int K, int rows) {
  // smallest power of two giving >= 2048 wave units, an LDS A chunk <= 48 KiB and >= 4 k-steps
  int ks = 1;
  while (true) {
    const int KC = K / ks;
    const bool lds_ok = (size_t)rows * (KC + 8) * 2 <= 48 * 1024;
    const bool units_ok = (long long)nex_units * tiles * ks >= 2048;
    if (lds_ok && units_ok) break;
    const int nks = ks * 2;
    if (K % (nks * 32) != 0 || K / nks < 128) break;
    ks = nks;
  }
  return ks;
}

size_t lds_bytes(int rows, int KC) { return (size_t)rows * (KC + 8) * 2; }

WS carve(const cfh_flow_dims* dm, char* base) {
  WS w;
  const size_t d = dm->d, fd = (size_t)dm->ffn_mult * dm->d;
  const int nch = dm->draft_length / dm->chunk_size;
  size_t off = 0;
  auto take = [&](size_t bytes) -> char* {
    char* p = base ? base + off : nullptr;
    off = cfh::align256(off + bytes);
    return p;
  };
  w.z = (float*)take(dm->draft_length * d * 4);
  for (int c = 0; c < nch; ++c) {
    const size_t S = (size_t)(c + 1) * dm->chunk_size;
    for (int p = 0; p < 2; ++p) {
      w.x[c][p] = (float*)take(S * d * 4);
      w.x16[c][p] = (h16*)take(S * d * 2);
    }
    w.qkv[c] = (h16*)take(S * 3 * d * 2);
    w.attn[c] = (h16*)take(S * d * 2);
    w.g[c] = (h16*)take(S * fd * 2);
    w.tau[c] = (h16*)take((size_t)dm->flow_steps * d * 2);
    w.kvc[c] = (h16*)take((size_t)dm->layers * 2 * dm->ctx_rows * d * 2);
  }
  w.ngen = 1 + (size_t)dm->flow_steps * (3 * dm->layers + 1);
  w.stats_floats = w.ngen * nch * MAXR * 2;
  w.stats = (float*)take(w.stats_floats * 4);
  // split-K partials and tile counters: launch_phase refuses a phase above MAX_UNITS per expert
  w.partial_floats = (size_t)nch * MAX_UNITS * 256;
  w.partials = (float*)take(w.partial_floats * 4);
  w.n_tile_ctr = (size_t)nch * MAX_UNITS;
  w.tile_ctr = (unsigned*)take(w.n_tile_ctr * 4);
  w.n_head_ctr = (size_t)nch * dm->heads;
  w.head_ctr = (unsigned*)take(w.n_head_ctr * 4);
  w.total = off;
  return w;
}

struct Ctx {
  const cfh_flow_dims* dm;
  cfh::ExpertLayout L;
  const char* ex[4];
  WS ws;
  int nch, d, fd, CS;
  hipStream_t st;
};

template <int KIND>
int launch_phase(PhaseArgs& a, int rows_max, hipStream_t st) {
  const int per_ex = a.nl * a.ksplit * a.tiles;
  const int units = a.nex * per_ex;
  if (a.tiles % WPB != 0) return CFH_E_UNSUPPORTED;
  if (a.ksplit > 1 && (size_t)a.nl * a.tiles * a.ksplit > (size_t)MAX_UNITS) return CFH_E_UNSUPPORTED;
  const size_t lds = lds_bytes(rows_max, a.K / a.ksplit);
  if (lds > 160 * 1024) return CFH_E_UNSUPPORTED;
  hipLaunchKernelGGL(k_phase<KIND>, dim3(units / WPB), dim3(WPB * 64), lds, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

}  // namespace

extern "C" {

int cfh_caps(const cfh_flow_dims* dims, int batch, int64_t* ws_bytes) {
  if (!cfh::flow_dims_ok(dims) || batch < 1) return CFH_E_UNSUPPORTED;
  const WS w = carve(dims, nullptr);
  if (ws_bytes) *ws_bytes = (int64_t)w.total;
  return CFH_OK;
}

int cfh_flow_integrate(const cfh_flow_dims* dm, const void* const* experts, const void* ctx, void* z_out,
                       void* ws_ptr, int batch, void* stream) {
  if (!cfh::flow_dims_ok(dm)) return CFH_E_UNSUPPORTED;
  if (!experts || !ctx || !z_out || !ws_ptr || batch < 1) return CFH_E_INVALID;
  const int nch = dm->draft_length / dm->chunk_size;
  for (int c = 0; c < nch; ++c)
    if (!experts[c]) return CFH_E_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const cfh::ExpertLayout L = cfh::expert_layout(dm);
  const WS w = carve(dm, (char*)ws_ptr);
  const int d = dm->d, fd = dm->ffn_mult * dm->d, CS = dm->chunk_size, E = dm->flow_steps,
            NL = dm->layers, C = dm->ctx_rows, KD = dm->draft_length, H = dm->heads;
  const size_t gen_stride = (size_t)nch * MAXR * 2;
  auto stats_of = [&](size_t gen, int c) { return w.stats + gen * gen_stride + (size_t)c * MAXR * 2; };
  auto P = [&](int c, size_t off) { return (const char*)experts[c] + off; };

  for (int b = 0; b < batch; ++b) {
    const h16* ctx_b = (const h16*)ctx + (size_t)b * C * d;
    h16* zo_b = (h16*)z_out + (size_t)b * KD * d;

    // ---- cross K/V (once per draft) and time embeddings (once per draft)
    {
      PhaseArgs a = {};
      a.nex = nch;
      a.nl = NL;
      a.wstride = (long long)L.blkstride;
      a.vstride = (long long)L.blkstride;
      a.d = d; a.N = 2 * d; a.K = d; a.tiles = 2 * d / 16; a.heads = H; a.hd = d / H; a.CS = CS; a.C = C;
      a.E = E; a.FD = fd; a.ctx = ctx_b;
      a.ksplit = 1;
      for (int c = 0; c < nch; ++c) {
        PhaseEx& x = a.ex[c];
        x.w = (const h16x8*)P(c, L.blk0 + L.kv);
        x.bias = (const h16*)P(c, L.blk0 + L.kv_b);
        x.lng = (const h16*)P(c, L.blk0 + L.cn_w);
        x.lnb = (const h16*)P(c, L.blk0 + L.cn_b);
        x.out = w.kvc[c];
        x.rows = C;
      }
      int rc = launch_phase<K_KV>(a, C, st);
      if (rc) return rc;
    }
    {
      PhaseArgs a = {};
      a.nex = nch; a.nl = 1;
      a.d = d; a.N = d; a.K = d; a.tiles = d / 16; a.heads = H; a.hd = d / H; a.CS = CS; a.C = C; a.E = E;
      a.FD = fd;
      a.ksplit = ksplit_for(nch, a.tiles, d, E);
      a.partials = w.partials; a.tile_ctr = w.tile_ctr;
      for (int c = 0; c < nch; ++c) {
        PhaseEx& x = a.ex[c];
        x.w = (const h16x8*)P(c, L.tw2);
        x.bias = (const h16*)P(c, L.tb2);
        x.lng = (const h16*)P(c, L.tw0);
        x.lnb = (const h16*)P(c, L.tb0);
        x.out = w.tau[c];
        x.rows = E;
      }
      // counters must be zero before the tau phase: init clears them, so run init first
      InitArgs ia = {};
      ia.ctx = ctx_b; ia.z = w.z; ia.d = d; ia.C = C; ia.KD = KD; ia.CS = CS; ia.nch = nch; ia.init_mode = 0;
      for (int c = 0; c < nch; ++c) {
        ia.x[c] = w.x[c][0]; ia.x16[c] = w.x16[c][0]; ia.st0[c] = stats_of(0, c);
        ia.pos[c] = (const h16*)P(c, L.pos); ia.tau0[c] = w.tau[c]; ia.srows[c] = (c + 1) * CS;
      }
      ia.zero_f = w.stats + gen_stride;
      ia.nzero_f = w.stats_floats - gen_stride;
      ia.zero_u = w.tile_ctr;
      ia.nzero_u = (size_t)((char*)(w.head_ctr + w.n_head_ctr) - (char*)w.tile_ctr) / 4;
      // tau needs clean counters; init needs tau.  Clear counters with a zero-only init pass
      // (no rows), run tau, then run the real init.
      InitArgs zc = ia;
      zc.nch = 0;
      hipLaunchKernelGGL(k_flow_init, dim3(KD), dim3(256), 0, st, zc);
      CFH_LAUNCH_CHECK();
      int rc = launch_phase<K_TAU>(a, E, st);
      if (rc) return rc;
      ia.zero_f = nullptr; ia.nzero_f = 0; ia.zero_u = nullptr; ia.nzero_u = 0;
      hipLaunchKernelGGL(k_flow_init, dim3(KD), dim3(256), 0, st, ia);
      CFH_LAUNCH_CHECK();
    }

    // ---- Euler steps
    size_t gen = 0;
    for (int s = 0; s < E; ++s) {
      for (int l = 0; l < NL; ++l) {
        const size_t B = L.blk0 + (size_t)l * L.blkstride;
        PhaseArgs a = {};
        a.nex = nch; a.nl = 1; a.d = d; a.heads = H; a.hd = d / H; a.CS = CS; a.C = C; a.E = E; a.FD = fd;
        a.partials = w.partials; a.tile_ctr = w.tile_ctr; a.head_ctr = w.head_ctr;
        for (int c = 0; c < nch; ++c) {
          PhaseEx& x = a.ex[c];
          x.x = w.x[c][s & 1]; x.x16 = w.x16[c][s & 1]; x.qkv = w.qkv[c]; x.attn = w.attn[c]; x.g = w.g[c];
          x.kv = w.kvc[c] + (size_t)l * 2 * C * d;
          x.rows = (c + 1) * CS; x.row0 = 0; x.srows = x.rows;
        }
        int rc;
        // QKV
        a.N = 3 * d; a.K = d; a.tiles = 3 * d / 16; a.ksplit = ksplit_for(nch, a.tiles, d, KD);
        for (int c = 0; c < nch; ++c) {
          PhaseEx& x = a.ex[c];
          x.w = (const h16x8*)P(c, B + L.qkv); x.bias = (const h16*)P(c, B + L.qkv_b);
          x.lng = (const h16*)P(c, B + L.sn_w); x.lnb = (const h16*)P(c, B + L.sn_b);
          x.st_in = stats_of(gen, c);
        }
        if ((rc = launch_phase<K_QKV>(a, KD, st))) return rc;
        // O
        a.N = d; a.K = d; a.tiles = d / 16; a.ksplit = ksplit_for(nch, a.tiles, d, KD);
        for (int c = 0; c < nch; ++c) {
          PhaseEx& x = a.ex[c];
          x.w = (const h16x8*)P(c, B + L.o); x.bias = (const h16*)P(c, B + L.o_b);
          x.st_out = stats_of(gen + 1, c);
        }
        if ((rc = launch_phase<K_O>(a, KD, st))) return rc;
        // QC
        a.N = d; a.K = d; a.tiles = d / 16; a.ksplit = ksplit_for(nch, a.tiles, d, KD);
        for (int c = 0; c < nch; ++c) {
          PhaseEx& x = a.ex[c];
          x.w = (const h16x8*)P(c, B + L.qc); x.bias = (const h16*)P(c, B + L.qc_b);
          x.lng = (const h16*)P(c, B + L.xn_w); x.lnb = (const h16*)P(c, B + L.xn_b);
          x.st_in = stats_of(gen + 1, c);
        }
        if ((rc = launch_phase<K_QC>(a, KD, st))) return rc;
        // OC
        for (int c = 0; c < nch; ++c) {
          PhaseEx& x = a.ex[c];
          x.w = (const h16x8*)P(c, B + L.oc); x.bias = (const h16*)P(c, B + L.oc_b);
          x.st_out = stats_of(gen + 2, c);
        }
        if ((rc = launch_phase<K_OC>(a, KD, st))) return rc;
        // W1
        a.N = fd; a.K = d; a.tiles = fd / 16; a.ksplit = ksplit_for(nch, a.tiles, d, KD);
        for (int c = 0; c < nch; ++c) {
          PhaseEx& x = a.ex[c];
          x.w = (const h16x8*)P(c, B + L.w1); x.bias = (const h16*)P(c, B + L.w1_b);
          x.lng = (const h16*)P(c, B + L.fn_w); x.lnb = (const h16*)P(c, B + L.fn_b);
          x.st_in = stats_of(gen + 2, c);
        }
        if ((rc = launch_phase<K_W1>(a, KD, st))) return rc;
        // W2
        a.N = d; a.K = fd; a.tiles = d / 16; a.ksplit = ksplit_for(nch, a.tiles, fd, KD);
        for (int c = 0; c < nch; ++c) {
          PhaseEx& x = a.ex[c];
          x.w = (const h16x8*)P(c, B + L.w2); x.bias = (const h16*)P(c, B + L.w2_b);
          x.st_out = stats_of(gen + 3, c);
        }
        if ((rc = launch_phase<K_W2>(a, KD, st))) return rc;
        gen += 3;
      }
      // OUT: velocity of the current chunk rows, Euler update, next step's pre_blocks rows
      PhaseArgs a = {};
      a.nex = nch; a.nl = 1; a.d = d; a.heads = H; a.hd = d / H; a.CS = CS; a.C = C; a.E = E; a.FD = fd;
      a.N = d; a.K = d; a.tiles = d / 16; a.ksplit = ksplit_for(nch, a.tiles, d, CS);
      a.partials = w.partials; a.tile_ctr = w.tile_ctr; a.head_ctr = w.head_ctr;
      a.dt = 1.0f / (float)E;
      a.has_next = (s + 1 < E);
      a.z = w.z; a.z_out = zo_b;
      for (int c = 0; c < nch; ++c) {
        PhaseEx& x = a.ex[c];
        x.w = (const h16x8*)P(c, L.out); x.bias = (const h16*)P(c, L.out_b);
        x.lng = (const h16*)P(c, L.on_w); x.lnb = (const h16*)P(c, L.on_b);
        x.st_in = stats_of(gen, c);
        x.x = w.x[c][s & 1]; x.x16 = w.x16[c][s & 1];
        x.x_next = w.x[c][(s + 1) & 1]; x.x16_next = w.x16[c][(s + 1) & 1];
        x.rows = CS; x.row0 = c * CS; x.srows = (c + 1) * CS;
        x.pos = (const h16*)P(c, L.pos);
        x.tau_next = w.tau[c] + (size_t)(s + 1 < E ? s + 1 : s) * d;
        x.st_next = stats_of(gen + 1, c);
      }
      int rc = launch_phase<K_OUT>(a, CS, st);
      if (rc) return rc;
      gen += 1;
    }
  }
  return CFH_OK;
}

}  // extern "C"
