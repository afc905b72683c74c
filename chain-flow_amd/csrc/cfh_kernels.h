// Generic kernels shared by the flow and the draft head: the split-K weight-streaming GEMV, the
// partial reductions and the row helpers.  Everything sits in an anonymous namespace, so each
// translation unit that includes this header owns its private copy of the kernels.
#pragma once
#include <algorithm>

#include "cfh_common.h"
#include "cfh_host.h"

namespace {

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also waits for every global
// load the wave has in flight (its release fence covers global memory), which would drain a
// weight prefetch issued before the barrier; this one waits for the LDS queue alone.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Copy rows x 8-half vectors from global to LDS with SB loads in flight per thread: every load of a
// batch is issued before the first LDS store, so the staging costs one memory round trip per batch
// instead of one per vector.
constexpr int SB = 8;

template <typename Src, typename Dst>
__device__ __forceinline__ void batched_copy(int total, Src src, Dst dst) {
  for (int base = 0; base < total; base += SB * (int)blockDim.x) {
    h16x8 t[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int idx = base + u * (int)blockDim.x + (int)threadIdx.x;
      if (idx < total) t[u] = src(idx);
    }
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int idx = base + u * (int)blockDim.x + (int)threadIdx.x;
      if (idx < total) dst(idx, t[u]);
    }
  }
}

constexpr int WPB = 4;            // waves per GEMV workgroup
constexpr int PF = 8;             // fragment loads in flight per wave
constexpr int MAXR = 16;          // max activation rows per expert (draft_length, ctx rows, steps)
constexpr int ROWT = 1024;        // threads of the row kernels (NORM / ROWS)
constexpr int ROWE = 16;          // max elements per thread in the row kernels (d <= 16384)
constexpr float LN_EPS = 1e-5f;

enum Src { SRC_BUF = 0, SRC_CTX, SRC_TAU, SRC_GATHER };

// The MFMA operand image of an [S][N] fp16 block (S <= 16 rows): the 8 values (r, 32 s + 8 g .. +7)
// of row r, which one lane of a 16x16x32 MFMA takes for k-step s and k-group g, form vector
// (4 s + g) S + r.  A wave's load of one k-step then reads 4 S contiguous 16-byte vectors, one per
// live lane, instead of 64-byte pieces of S rows a row apart.
__host__ __device__ __forceinline__ size_t frag_index(int r, int n, int S) {
  return (((size_t)(n >> 5) * 4 + ((n >> 3) & 3)) * S + r) * 8 + (n & 7);
}

// ---------------------------------------------------------------------------- GEMV
struct GemvEx {
  const h16x8* w;      // packed weight fragments (layer 0 when nl > 1)
  const h16* a;        // SRC_BUF: activation rows [rows][lda]; SRC_CTX: context rows [rows][K]
  int lda;
  const h16* g0;       // SRC_CTX: context_norm weight (layer 0) | SRC_TAU: time_mlp.0.weight
  const h16* b0;       // SRC_CTX: context_norm bias             | SRC_TAU: time_mlp.0.bias
  float* pout;         // partial outputs [(l*ks + kc)][rows][N]
  const float* mom;    // SRC_CTX: context row moments [rows][2] = (mean, rstd)
  const int* ids;      // SRC_GATHER: row i of A = a[max(ids[i * ids_stride], 0)] (a row-major, lda)
  int ids_stride;
  int rows;
  h16* hout;           // ks == 1: out = fp16(acc + hb) written here instead of partials (the
  const h16* hb;       // partial reduce's arithmetic), hb layer l at + l * vstride bytes
};

constexpr int MAXEX = 8;          // weight sets (experts / path offsets) per GEMV launch

struct GemvArgs {
  GemvEx ex[MAXEX];
  int nex, nl, ks, tiles, N, K, E;
  long long wstride, vstride;   // bytes between consecutive layers (packed weights / vectors)
  int kvout;                    // hout layout: 0 [l][rows][N], 1 [l][2][rows][N/2] (cross K | V)
};

template <int SRC>
__device__ void stage_A(const GemvArgs& a, const GemvEx& ep, int l, int kc, h16* As, int lda) {
  const int KC = a.K / a.ks;
  const int k0 = kc * KC;
  const int rows = ep.rows;
  const int nvec = KC / 8;
  if constexpr (SRC == SRC_BUF) {
    batched_copy(rows * nvec,
                 [&](int idx) {
                   const int i = idx / nvec, kk = (idx - i * nvec) * 8;
                   return *(const h16x8*)(ep.a + (size_t)i * ep.lda + k0 + kk);
                 },
                 [&](int idx, h16x8 v) {
                   const int i = idx / nvec, kk = (idx - i * nvec) * 8;
                   *(h16x8*)(As + i * lda + kk) = v;
                 });
  } else if constexpr (SRC == SRC_GATHER) {
    batched_copy(rows * nvec,
                 [&](int idx) {
                   const int i = idx / nvec, kk = (idx - i * nvec) * 8;
                   const int id = max(ep.ids[i * ep.ids_stride], 0);
                   return *(const h16x8*)(ep.a + (size_t)id * ep.lda + k0 + kk);
                 },
                 [&](int idx, h16x8 v) {
                   const int i = idx / nvec, kk = (idx - i * nvec) * 8;
                   *(h16x8*)(As + i * lda + kk) = v;
                 });
  } else if constexpr (SRC == SRC_CTX) {
    // context_norm(ctx) of layer l; the row moments (mean, rstd) come precomputed in ep.mom
    const h16* gw = (const h16*)((const char*)ep.g0 + (size_t)l * a.vstride);
    const h16* gb = (const h16*)((const char*)ep.b0 + (size_t)l * a.vstride);
    for (int idx = threadIdx.x; idx < rows * nvec; idx += blockDim.x) {
      const int i = idx / nvec, kk = (idx - i * nvec) * 8;
      const h16x8 xv = *(const h16x8*)(ep.a + (size_t)i * a.K + k0 + kk);
      const h16x8 gv = *(const h16x8*)(gw + k0 + kk);
      const h16x8 bv = *(const h16x8*)(gb + k0 + kk);
      const float mu = ep.mom[2 * i], rs = ep.mom[2 * i + 1];
      h16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (h16)(((float)xv[e] - mu) * rs * (float)gv[e] + (float)bv[e]);
      *(h16x8*)(As + i * lda + kk) = o;
    }
  } else if constexpr (SRC == SRC_TAU) {
    // rows = Euler steps: a_s = fp16(silu(fp16(tau_s * w0 + b0))), tau_s = fp16(s / E)
    for (int idx = threadIdx.x; idx < rows * nvec; idx += blockDim.x) {
      const int i = idx / nvec, kk = (idx - i * nvec) * 8;
      const float tau = r16((float)i * (1.0f / (float)a.E));
      h16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float h = r16(tau * (float)ep.g0[k0 + kk + e] + (float)ep.b0[k0 + kk + e]);
        o[e] = (h16)silu(h);
      }
      *(h16x8*)(As + i * lda + kk) = o;
    }
  }
  __syncthreads();
}

template <int SRC>
__global__ void __launch_bounds__(WPB * 64) k_gemv(GemvArgs a) {
  extern __shared__ __align__(16) h16 As[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int per_ex = a.nl * a.ks * a.tiles;
  const int u0 = blockIdx.x * WPB;
  const int e = u0 / per_ex;
  int rem = u0 - e * per_ex;
  const int l = rem / (a.ks * a.tiles);
  rem -= l * a.ks * a.tiles;
  const int kc = rem / a.tiles;
  const int t = wave + (rem - kc * a.tiles);   // a workgroup never straddles (e, l, kc)
  const GemvEx& ep = a.ex[e];
  const int KC = a.K / a.ks;
  const int lda = KC + 8;

  // The weight stream does not depend on the activations: put its first PF fragment loads in
  // flight before staging the activation chunk.
  const h16x8* wbase = (const h16x8*)((const char*)ep.w + (size_t)l * a.wstride);
  TileStream<PF> ts;
  ts.begin(wbase + packed_index(t, kc * (KC / 32), a.K, 0), KC / 32);
  stage_A<SRC>(a, ep, l, kc, As, lda);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = ts.run(As, lda, ep.rows, acc);

  const int col = lane & 15, rbase = 4 * (lane >> 4);
  if (ep.hout) {
    const int n = t * 16 + col;
    const float b = (float)((const h16*)((const char*)ep.hb + (size_t)l * a.vstride))[n];
    const int half = a.N / 2, part = a.kvout ? n / half : 0, nn = a.kvout ? n - part * half : n;
    const int ld = a.kvout ? half : a.N;
    h16* ho = ep.hout + ((size_t)(l * (a.kvout ? 2 : 1) + part) * ep.rows) * ld + nn;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (rbase + j < ep.rows) ho[(size_t)(rbase + j) * ld] = (h16)(acc[j] + b);
    return;
  }
  float* po = ep.pout + ((size_t)(l * a.ks + kc) * ep.rows) * a.N + t * 16 + col;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (rbase + j < ep.rows) po[(size_t)(rbase + j) * a.N] = acc[j];
}

// ---------------------------------------------------------------------------- partial reduce
// out = fp16(sum_kc P[kc] + b), used for split-K cross K/V rows and the packed time embeddings;
// with act = 1, out = fp16(silu(fp16(sum_kc P[kc] + b))) (a Linear module then a SiLU module, as the
// anchor MLP).
struct ReduceArgs {
  const float* P[4];
  const h16* b[4];
  h16* out[4];
  int nex, nl, ks, rows, N, d, kv;   // kv: N = 2d split into [2][rows][d] per layer
  int act;
  long long vstride;
};

__global__ void __launch_bounds__(256) k_reduce(ReduceArgs a) {
  const size_t per_l = (size_t)a.rows * a.N;
  const size_t per_e = per_l * a.nl;
  const size_t total = per_e * a.nex;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int e = (int)(i / per_e);
    size_t r = i - e * per_e;
    const int l = (int)(r / per_l);
    r -= (size_t)l * per_l;
    const int row = (int)(r / a.N), n = (int)(r - (size_t)row * a.N);
    const float* P = a.P[e] + (size_t)l * a.ks * per_l + (size_t)row * a.N + n;
    float s = 0.f;
    for (int q = 0; q < a.ks; ++q) s += P[(size_t)q * per_l];
    const h16* b = (const h16*)((const char*)a.b[e] + (size_t)l * a.vstride);
    float v = s + (float)b[n];
    if (a.act == 1) v = silu(r16(v));
    size_t o;
    if (a.kv) {
      const int part = n / a.d, nn = n - part * a.d;
      o = (((size_t)l * 2 + part) * a.rows + row) * a.d + nn;
    } else {
      o = ((size_t)l * a.rows + row) * a.N + n;
    }
    a.out[e][o] = (h16)v;
  }
}

// ---------------------------------------------------------------------------- GELU
// g = fp16(gelu(fp16(sum_kc P[kc] + b1))) for every row of every expert: the sum is rounded to fp16
// first, as torch's fp16 Linear module hands its output to the GELU module.
struct GeluArgs {
  const float* P[4];
  const h16* b[4];
  h16* g[4];
  int rows[4];
  int nex, ks, N;
};

__global__ void __launch_bounds__(256) k_gelu(GeluArgs a) {
  size_t total = 0;
  for (int e = 0; e < a.nex; ++e) total += (size_t)a.rows[e] * a.N / 4;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    int e = 0;
    size_t j = i;
    while (j >= (size_t)a.rows[e] * a.N / 4) j -= (size_t)a.rows[e++] * a.N / 4;
    const size_t per_kc = (size_t)a.rows[e] * a.N;
    const float* P = a.P[e] + j * 4;
    float4 s4 = *(const float4*)P;
    for (int q = 1; q < a.ks; ++q) {
      const float4 t = *(const float4*)(P + q * per_kc);
      s4.x += t.x; s4.y += t.y; s4.z += t.z; s4.w += t.w;
    }
    const int n = (int)((j * 4) % a.N);
    const h16* bb = a.b[e] + n;
    h16* g = a.g[e] + j * 4;
    g[0] = (h16)gelu_erf(r16(s4.x + (float)bb[0]));
    g[1] = (h16)gelu_erf(r16(s4.y + (float)bb[1]));
    g[2] = (h16)gelu_erf(r16(s4.z + (float)bb[2]));
    g[3] = (h16)gelu_erf(r16(s4.w + (float)bb[3]));
  }
}

// ---------------------------------------------------------------------------- row kernels
// Block-wide sum over the workgroup.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  lds_barrier();   // (not __syncthreads: no wait for the row's global stores in flight)
  if (lane == 0) red[wave] = v;
  lds_barrier();
  float t = 0.f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += red[w];
  return t;
}

// LayerNorm of one row held as fp16-valued floats: thread t owns the float4 column groups
// t, t + blockDim, ... (vals[k] = group k); two-pass moments; fp16 output.
constexpr int ROWQ = ROWE / 4;   // float4 groups per thread

template <int RQ = ROWQ>
__device__ void ln_row4(const float4* vals, int d, const h16* g, const h16* b, h16* out, float* red) {
  const int nq = d / 4;
  // gamma and beta are loaded before the statistics, not after them
  h16x4 gq[RQ], bq[RQ];
#pragma unroll
  for (int k = 0; k < RQ; ++k) {
    const int q = threadIdx.x + k * blockDim.x;
    if (q < nq) {
      gq[k] = *(const h16x4*)(g + q * 4);
      bq[k] = *(const h16x4*)(b + q * 4);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < RQ; ++k) {
    const int q = threadIdx.x + k * blockDim.x;
    if (q < nq) s += (vals[k].x + vals[k].y) + (vals[k].z + vals[k].w);
  }
  const float mean = block_sum(s, red) / (float)d;
  float v = 0.f;
#pragma unroll
  for (int k = 0; k < RQ; ++k) {
    const int q = threadIdx.x + k * blockDim.x;
    if (q < nq) {
      const float a0 = vals[k].x - mean, a1 = vals[k].y - mean, a2 = vals[k].z - mean, a3 = vals[k].w - mean;
      v += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
    }
  }
  const float rstd = 1.0f / sqrtf(block_sum(v, red) / (float)d + LN_EPS);
#pragma unroll
  for (int k = 0; k < RQ; ++k) {
    const int q = threadIdx.x + k * blockDim.x;
    if (q < nq) {
      h16x4 o;
      o[0] = (h16)((vals[k].x - mean) * rstd * (float)gq[k][0] + (float)bq[k][0]);
      o[1] = (h16)((vals[k].y - mean) * rstd * (float)gq[k][1] + (float)bq[k][1]);
      o[2] = (h16)((vals[k].z - mean) * rstd * (float)gq[k][2] + (float)bq[k][2]);
      o[3] = (h16)((vals[k].w - mean) * rstd * (float)gq[k][3] + (float)bq[k][3]);
      *(h16x4*)(out + q * 4) = o;
    }
  }
}

__device__ __forceinline__ float4 r16x4(float4 v) { return make_float4(r16(v.x), r16(v.y), r16(v.z), r16(v.w)); }

size_t lds_bytes(int rows, int KC) { return (size_t)rows * (KC + 8) * 2; }

// Split-K factor: the smallest divisor ks of the k-step count such that every unit streams a
// whole number of PF-step prefetch blocks, the A chunk fits in 48 KiB of LDS (two or three
// workgroups per CU) and the phase has >= 2048 wave units; else the largest valid one.
int ksplit_for(int nex_units, int tiles, int K, int rows) {
  const int steps = K / 32;
  int best = -1;
  for (int ks = 1; ks <= steps; ++ks) {
    if (steps % ks) continue;
    if ((steps / ks) % PF) continue;
    if (lds_bytes(rows, K / ks) > 48 * 1024) continue;
    best = ks;
    if ((long long)nex_units * tiles * ks >= 2048) break;
  }
  if (best > 0) return best;
  for (int ks = 1; ks <= steps; ++ks)
    if (steps % ks == 0 && lds_bytes(rows, K / ks) <= 48 * 1024) return ks;
  return steps;
}

template <int SRC>
int launch_gemv(const GemvArgs& a, int rows_max, hipStream_t st) {
  if (a.tiles % WPB != 0) return CFH_E_UNSUPPORTED;
  for (int e = 0; e < a.nex; ++e)
    if (a.ex[e].hout && a.ks != 1) return CFH_E_UNSUPPORTED;   // direct output needs the whole K
  const size_t lds = lds_bytes(rows_max, a.K / a.ks);
  if (lds > 64 * 1024) return CFH_E_UNSUPPORTED;
  const long long units = (long long)a.nex * a.nl * a.ks * a.tiles;
  hipLaunchKernelGGL(k_gemv<SRC>, dim3((unsigned)(units / WPB)), dim3(WPB * 64), lds, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

}  // namespace
