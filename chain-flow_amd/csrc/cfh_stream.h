// The weight-streaming GEMM kernel with its operand staging (plain rows, or self / cross attention
// computed while the weights stream) and the residual + LayerNorm row kernel, shared by the flow
// (flow.hip) and the hidden-state VAE (vae.hip).  Everything sits in an anonymous namespace: each
// translation unit that includes this header owns its private copy of the kernels.
//
// Streaming kernel: a wave owns TPW consecutive 16-column tiles of one (expert, k-chunk); it
// streams their packed fragments (1 KiB per wave per k-step, contiguous per tile, non-temporal)
// with PF fragment loads in flight, issued before the A operand is staged, and multiplies each
// against the A rows held in LDS with v_mfma_f32_16x16x32_f16.
#pragma once
#include <algorithm>

#include "cfh_kernels.h"

namespace {

constexpr int SWMAX = 16;         // max waves per streaming workgroup
constexpr int PF_FULL = 16;       // fragment loads in flight per wave: full-K kernels
constexpr int PF_SPLIT = 8;       //                                   split-K kernels
constexpr int STREAM_SYNC = 4;    // fragment groups between workgroup barriers in the stream (measured: 4 best of 0-4)

enum SrcKind { S_BUF = 0, S_SELF = 1, S_CROSS = 2 };
enum EpiKind { E_PART = 0, E_BIAS16 = 1, E_GELU16 = 2, E_PART16 = 3 };

struct SEx {
  const h16x8* w;      // packed weights: fragment (tile t, k-step s) at ((t * K/32) + s) * 64
  const h16* a;        // S_BUF: rows [S][lda] | S_SELF: q,k,v rows [S][3d] | S_CROSS: K/V [2][Ck][d]
  int lda;
  const float* pin;    // S_CROSS: cross-q partials [ks_in][S][d]
  const h16* bin;      // S_CROSS: cross-q bias (in_proj_bias[0:d])
  const h16* bias;     // E_BIAS16 / E_GELU16 bias [N]
  void* out;           // E_PART: float [ks][S][N]; E_PART16: h16 [ks][S][N]; otherwise h16 [S][N]
  int S;               // activation rows (<= 16)
  int Sr;              // S_SELF / S_CROSS: rows per request (requests packed in the S rows; 0 = S)
  int pack;            // E_PART16: each k-chunk's [S][N] block in frag_index order
  int hrows;           // E_PART16: rows per output block (0 = S): row r of k-chunk kc goes to block
                       // kc * (S / hrows) + r / hrows, as its row r % hrows
};

// For the attention kinds a k-chunk of KC = K / ks columns holds KC / hd whole heads (one head
// when hd is a multiple of 32; two for head widths such as 80 or 240).
struct SArgs {
  SEx ex[4];
  int nex, N, K, ks, wpb, tpw, wg_per_kc;
  int d, hd, ks_in, Ck;
  int Cr;              // S_CROSS: context rows per request (the Ck rows hold Ck / Cr requests; 0 = Ck)
  int sync;            // fragment groups between workgroup barriers in the stream (0: none)
  int causal;          // S_SELF: causal mask triu(-inf, 1) (the flow's draft rows) or none
  int gelu_r16;        // E_GELU16: round acc + bias to fp16 before the GELU (a Linear module
                       // followed by a GELU module) instead of once after it (the fused block)
  int conc;            // launches of this shape running concurrently (one per chunk expert's stream)
  // E_PART16 only: nl layers in one launch, layer l's entries at the same pointers advanced by
  // l * (lwb, lab, lob) bytes (weights, operand rows, output)
  int nl;
  long long lwb, lab, lob;
};

// LDS that concurrent streaming launches reserve when together they fit one workgroup a CU:
// above half a CU's LDS, so their workgroups spread over the CUs.  Left to share, the two experts'
// workgroups pile onto the CUs where they fit twice while other CUs idle (d = 2560: 7.92 against
// 7.52 ms a flow pass reserved); when they do not fit one a CU (d = 1024), sharing is better
// (3.97 against 4.48 ms), and where one a CU is the most that fits anyway (d = 5120) it is neutral.
constexpr size_t CONC_LDS = 82 * 1024;

// Attention of the KC / hd heads of a k-chunk for the S rows of one expert from q, k, v already in
// LDS (sq [S][KC], sk and sv [Sk][KC], Sk <= 16; head hh in columns [hh hd, hh hd + hd)), written
// as fp16 into As [S][lda].  Causal mask = triu(-inf, 1) (cf/drafters/chunked_flow.py:273-275);
// scores and the weighted sum in fp32 on fp16 q/k/v, output rounded to fp16.  Rows of several
// requests may share the tile: query row i belongs to request i / Sr and key j to request j / Cr,
// and a query attends only to its own request's keys (one request: Sr = S, Cr = Sk).
// One wave per (head, query row): lane group j (LP lanes) holds key j, so the dot products, the
// row max, exp and sum stay in registers (DPP reductions); every LDS read of a phase is issued
// before the first is used.  (A wave per (i, j) pair with a serial softmax thread per row spent
// 2-4 us here, almost all of it in dependent LDS round trips.)
__device__ void attend(int S, int Sk, int Sr, int Cr, int hd, int KC, bool causal, const h16* sq, const h16* sk,
                       const h16* sv, float* P, h16* As, int lda) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const int hpk = KC / hd;
  const float scale = 1.0f / sqrtf((float)hd);
  const bool l8 = Sk <= 8;                 // 8 lanes per key (else 4)
  const int j = l8 ? lane >> 3 : lane >> 2, sub = l8 ? lane & 7 : lane & 3;
  const int step = l8 ? 64 : 32;           // halves between a lane's 8-half chunks
  const int jr = min(j, Sk - 1);           // lanes of keys >= Sk read a valid row, result masked
  for (int ri = wave; ri < hpk * S; ri += nw) {
    const int hh = ri / S, i = ri - hh * S;
    const h16* qr = sq + i * KC + hh * hd;
    const h16* kr = sk + jr * KC + hh * hd;
    float part = 0.f;
    for (int c = sub * 8; c < hd; c += step) {
      const h16x8 qa = *(const h16x8*)(qr + c);
      const h16x8 kb = *(const h16x8*)(kr + c);
#pragma unroll
      for (int t = 0; t < 8; ++t) part += (float)qa[t] * (float)kb[t];
    }
    part += dpp_f32<DPP_XOR1>(part);
    part += dpp_f32<DPP_XOR2>(part);
    if (l8) part += dpp_f32<DPP_HMIRROR>(part);
    const bool valid = j < Sk && j / Cr == i / Sr && !(causal && j > i);
    const float sc = valid ? part * scale : -INFINITY;
    const float m = wave_max(sc);
    const float e = valid ? expf(sc - m) : 0.f;
    const float inv = 1.0f / wave_sum(sub == 0 ? e : 0.f);
    if (sub == 0 && j < Sk) P[ri * Sk + j] = e * inv;
  }
  lds_barrier();
  const int nv = hd / 8;
  for (int idx = threadIdx.x; idx < hpk * S * nv; idx += blockDim.x) {
    const int ri = idx / nv, c = (idx - ri * nv) * 8;
    const int hh = ri / S, i = ri - hh * S;
    const h16* vh = sv + hh * hd + c;
    float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j0 = 0; j0 < Sk; j0 += 8) {   // 8 keys at a time; keys past Sk: a valid row, weight 0
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int jc = min(j0 + jj, Sk - 1);
        const float p = j0 + jj < Sk ? P[ri * Sk + jc] : 0.f;
        const h16x8 vb = *(const h16x8*)(vh + jc * KC);
#pragma unroll
        for (int t = 0; t < 8; ++t) o[t] += p * (float)vb[t];
      }
    }
    h16x8 ov;
#pragma unroll
    for (int t = 0; t < 8; ++t) ov[t] = (h16)o[t];
    *(h16x8*)(As + i * lda + hh * hd + c) = ov;
  }
}

// Operand staging in two phases around the weight prefetch.  A wave's vector loads complete in
// issue order, so operand loads issued after the prefetch burst would wait for all of it; instead
// `load` issues every operand load of the thread (at most NS, which the launcher guarantees) into
// registers, the kernel then puts the weight prefetch in flight, and `place` writes the registers
// to LDS.  There is deliberately no slower path for operands that do not fit: its loads would
// make the compiler's wait before the first multiply cover the whole prefetch.
// Every slot load and store is unconditional, its index clamped into range (a clamped slot
// rewrites the last vector with the value it holds), so that the compiler cannot sink a load past
// the prefetch into a conditional store, where the wait before the store would cover the prefetch.
//   S_BUF  : vectors idx = u * nt + t of the A chunk [S][KC] -> As [S][lda]
//   S_SELF : vectors of the q | k | v columns of the k-chunk (each [S][KC]) -> consecutive LDS
//            blocks sq, sk, sv
//   S_CROSS: the ks_in fp32 partials of each 4-column q group g = t + j * nt the thread owns
//            (slot q * gj + j; summed in the order q = 0, 1, ...) and then the vectors of the
//            hoisted context K and V rows of the k-chunk's columns
template <int SRC, int NS>
struct Stage {
  h16x8 st[NS];
  int nqs;   // S_CROSS: q-partial slots (ks_in * gj)
  int gj;    // S_CROSS: q groups per thread (<= 4)
  uint2 qb[4];   // S_CROSS: the 4 fp16 q-bias values of each q group

  __device__ __forceinline__ static const h16x8* buf_src(const SEx& ex, int kc, int KC, int nv, int idx) {
    const int i = idx / nv, kk = (idx - i * nv) * 8;
    return (const h16x8*)(ex.a + (size_t)i * ex.lda + (size_t)kc * KC + kk);
  }
  __device__ __forceinline__ static const h16x8* self_src(const SArgs& a, const SEx& ex, int kc, int KC, int nv,
                                                         int idx) {
    const int part = idx / (ex.S * nv);
    const int r = idx - part * ex.S * nv;
    const int i = r / nv, c = (r - i * nv) * 8;
    return (const h16x8*)(ex.a + (size_t)i * 3 * a.d + part * a.d + kc * KC + c);
  }
  __device__ __forceinline__ static const h16x8* kv_src(const SArgs& a, const SEx& ex, int kc, int KC, int nv,
                                                       int idx) {
    const int j = idx / nv, c = (idx - j * nv) * 8;   // j < 2 Ck: K rows then V rows
    return (const h16x8*)(ex.a + (size_t)j * a.d + kc * KC + c);
  }
  __device__ __forceinline__ static const h16x8* q_src(const SArgs& a, const SEx& ex, int kc, int KC, int g, int q) {
    const int nq = KC / 4;
    const int i = g / nq, c = (g - i * nq) * 4;
    return (const h16x8*)(ex.pin + (size_t)q * ex.S * a.d + (size_t)i * a.d + kc * KC + c);
  }

  __device__ __forceinline__ void load(const SArgs& a, const SEx& ex, int kc, int KC) {
    const int t = threadIdx.x, nt = blockDim.x;
    if constexpr (SRC == S_BUF) {
      const int nv = KC / 8, total = ex.S * nv;
#pragma unroll
      for (int u = 0; u < NS; ++u) st[u] = *buf_src(ex, kc, KC, nv, min(u * nt + t, total - 1));
    } else if constexpr (SRC == S_SELF) {
      const int nv = KC / 8, total = 3 * ex.S * nv;
#pragma unroll
      for (int u = 0; u < NS; ++u) st[u] = *self_src(a, ex, kc, KC, nv, min(u * nt + t, total - 1));
    } else {
      const int nq = KC / 4, G = ex.S * nq, nv = KC / 8, nkv = 2 * a.Ck * nv;
      gj = (G + nt - 1) / nt;
      nqs = a.ks_in * gj;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int g = min(t + j * nt, G - 1);
        qb[j] = *(const uint2*)(ex.bin + kc * KC + (g - (g / nq) * nq) * 4);
      }
#pragma unroll
      for (int u = 0; u < NS; ++u) {
        if (u < nqs) {
          const int q = u / gj, j = u - q * gj;
          st[u] = *q_src(a, ex, kc, KC, min(t + j * nt, G - 1), q);
        } else {
          st[u] = *kv_src(a, ex, kc, KC, nv, min((u - nqs) * nt + t, nkv - 1));
        }
      }
    }
  }

  __device__ __forceinline__ void place(const SArgs& a, const SEx& ex, int kc, int KC, h16* As, int lda) {
    const int t = threadIdx.x, nt = blockDim.x;
    if constexpr (SRC == S_BUF) {
      const int nv = KC / 8, total = ex.S * nv;
      auto put = [&](int idx, h16x8 v) {
        const int i = idx / nv, kk = (idx - i * nv) * 8;
        *(h16x8*)(As + i * lda + kk) = v;
      };
#pragma unroll
      for (int u = 0; u < NS; ++u) put(min(u * nt + t, total - 1), st[u]);
      lds_barrier();
    } else {
      const int S = ex.S, nv = KC / 8;
      const int Sk = SRC == S_SELF ? S : a.Ck;
      h16* sq = As + (size_t)S * lda;
      h16* sk = sq + (size_t)S * KC;
      h16* sv = sk + (size_t)Sk * KC;
      float* P = (float*)(sv + (size_t)Sk * KC);   // [KC / hd][S][Sk]
      if constexpr (SRC == S_SELF) {
        const int total = 3 * S * nv;
#pragma unroll
        for (int u = 0; u < NS; ++u) *(h16x8*)(sq + (size_t)min(u * nt + t, total - 1) * 8) = st[u];
      } else {
        const int nq = KC / 4, G = S * nq, nkv = 2 * Sk * nv;
        // q = fp16(sum of the cross-q partials + bias) for the 4-column group g
        auto put_q = [&](int g, float4 s4, uint2 bw) {
          const int i = g / nq, c = (g - i * nq) * 4;
          const h16x4 bb = __builtin_bit_cast(h16x4, bw);
          h16* dst = sq + i * KC + c;
          dst[0] = (h16)(s4.x + (float)bb[0]);
          dst[1] = (h16)(s4.y + (float)bb[1]);
          dst[2] = (h16)(s4.z + (float)bb[2]);
          dst[3] = (h16)(s4.w + (float)bb[3]);
        };
        auto add4 = [](float4& s4, float4 v) { s4.x += v.x; s4.y += v.y; s4.z += v.z; s4.w += v.w; };
        float4 qs[4] = {};
#pragma unroll
        for (int u = 0; u < NS; ++u) {
          if (u < nqs) {
            const int q = u / gj, j = u - q * gj;
            const float4 v = __builtin_bit_cast(float4, st[u]);
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
              if (jj == j) {
                if (q == 0) qs[jj] = v;
                else add4(qs[jj], v);
              }
          } else {
            *(h16x8*)(sk + (size_t)min((u - nqs) * nt + t, nkv - 1) * 8) = st[u];
          }
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          if (jj < gj && t + jj * nt < G) put_q(t + jj * nt, qs[jj], qb[jj]);
      }
      lds_barrier();
      const int Sr = ex.Sr > 0 ? ex.Sr : S;
      const int Cr = SRC == S_SELF ? Sr : (a.Cr > 0 ? a.Cr : Sk);
      attend(S, Sk, Sr, Cr, a.hd, KC, SRC == S_SELF && a.causal, sq, sk, sv, P, As, lda);
      lds_barrier();
    }
  }
};

template <int SRC, int EPI, int SPF, int NS, int WV>
__global__ void __launch_bounds__(WV * 64) k_stream(SArgs a) {
  extern __shared__ __align__(16) h16 lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int b = blockIdx.x;
  const int per_ex = a.ks * a.wg_per_kc;
  int l = 0;
  if constexpr (EPI == E_PART16) {
    const int per_l = a.nex * per_ex;
    l = b / per_l;
    b -= l * per_l;
  }
  const int e = b / per_ex;
  b -= e * per_ex;
  const int kc = b / a.wg_per_kc;
  const int tg = b - kc * a.wg_per_kc;
  SEx exl;   // (E_PART16: layer l's copy of the entry; the other kinds read the entry in place)
  if constexpr (EPI == E_PART16) {
    exl = a.ex[e];
    exl.w = (const h16x8*)((const char*)exl.w + l * a.lwb);
    exl.a = (const h16*)((const char*)exl.a + l * a.lab);
    exl.out = (char*)exl.out + l * a.lob;
  }
  const SEx& ex = EPI == E_PART16 ? exl : a.ex[e];
  const int ksteps = a.K / 32;
  const int KC = a.K / a.ks, nsteps = KC / 32;
  const int t0 = (tg * a.wpb + wave) * a.tpw;
  const int nf = a.tpw * nsteps;
  const int lda = KC + 8;
  // Fragment loader: a wave-uniform pointer walked one fragment at a time (the next tile of the
  // wave starts ksteps - nsteps fragments further on); past the last fragment it stays there, so
  // the ring's surplus refills re-read a line just fetched.  Walking the pointer, rather than
  // deriving each address from the fragment index, keeps integer divisions out of the loop
  // (measured: they cost ~5% of the streaming rate).
  const h16x8* lw = ex.w + ((size_t)t0 * ksteps + (size_t)kc * nsteps) * 64;
  const size_t jump = (size_t)(ksteps - nsteps + 1) * 64;
  int ls = 0, lleft = nf;
  auto issue = [&]() -> h16x8 {
    const h16x8 v = __builtin_nontemporal_load(lw + lane);
    const bool adv = lleft > 1, wrap = ls == nsteps - 1;
    lw += adv ? (wrap ? jump : 64) : 0;
    ls = adv ? (wrap ? 0 : ls + 1) : ls;
    lleft -= adv;
    return v;
  };
  // operand loads first, then the weight prefetch (independent of the operand), then LDS
  // (the scheduling barriers keep the three groups in this order)
  Stage<SRC, NS> sg;
  sg.load(a, ex, kc, KC);
  // the bias of the wave's first tile comes with the operand: an epilogue load issued after the
  // weight loads would wait for every one of them
  float bias0 = 0.f;
  if constexpr (EPI == E_BIAS16 || EPI == E_GELU16) bias0 = (float)ex.bias[t0 * 16 + (lane & 15)];
  __builtin_amdgcn_sched_barrier(0);
  h16x8 buf[SPF];
#pragma unroll
  for (int p = 0; p < SPF; ++p) buf[p] = issue();
  __builtin_amdgcn_sched_barrier(0);
  h16* As = lds;
  sg.place(a, ex, kc, KC, As, lda);
  const int row = lane & 15, kg = lane >> 4;
  // lanes of padding rows (row >= S) read row 0: their products land only in output rows that
  // are never stored, so no zeroing is needed
  const h16* arow = As + (row < ex.S ? row : 0) * lda + kg * 8;
  const int col = lane & 15, rbase = 4 * (lane >> 4);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  // the next fragment to multiply is k-step cs of the wave's tile ct; the tile is stored after its
  // last k-step
  int cs = 0, ct = 0;
  auto step = [&](h16x8 bf) {
    const h16x8 av = *(const h16x8*)(arow + cs * 32);
    acc = mfma_f16(av, bf, acc);
    if (cs == nsteps - 1) {
      const int n = (t0 + ct) * 16 + col;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = rbase + q;
        if (r < ex.S) {
          if constexpr (EPI == E_PART) {
            ((float*)ex.out)[((size_t)kc * ex.S + r) * a.N + n] = acc[q];
          } else if constexpr (EPI == E_PART16) {
            const int hr = ex.hrows > 0 ? ex.hrows : ex.S, hb = r / hr, rr = r - hb * hr;
            h16* o = (h16*)ex.out + ((size_t)kc * (ex.S / hr) + hb) * hr * a.N;
            o[ex.pack ? frag_index(rr, n, hr) : (size_t)rr * a.N + n] = (h16)acc[q];
          } else {
            float bv;
            if (ct == 0) bv = bias0;
            else bv = (float)ex.bias[n];
            if constexpr (EPI == E_BIAS16) {
              ((h16*)ex.out)[(size_t)r * a.N + n] = (h16)(acc[q] + bv);
            } else {
              const float u = acc[q] + bv;
              ((h16*)ex.out)[(size_t)r * a.N + n] = (h16)gelu_erf(a.gelu_r16 ? r16(u) : u);
            }
          }
        }
      }
      acc = (f32x4){0.f, 0.f, 0.f, 0.f};
      ++ct;
      cs = 0;
    } else {
      ++cs;
    }
  };
  // Slot p is consumed and then refilled with the fragment SPF ahead, always, so the ring's
  // registers stay fixed across iterations and each multiply waits only for its own fragment.
  // A conditional refill would make the wait before every multiply cover all loads in flight, and
  // a separate drain after the loop makes the compiler copy the ring between registers at the
  // loop entry, which waits for the whole prefetch (both measured in the generated code).
  // Every a.sync groups the waves of the workgroup meet at a barrier (no memory fence: the rings
  // stay in flight).  Left alone, the oldest wave on each SIMD wins the issue arbitration and
  // finishes far ahead of the youngest (measured: 16-wave workgroups end spread over 35 us of a
  // 95 us stream), and the last third of the stream then runs with a fraction of the loads in
  // flight; in step, all waves finish together.
  int g = 0;
  for (int f0 = 0; f0 < nf; f0 += SPF) {
#pragma unroll
    for (int p = 0; p < SPF; ++p) {
      if (f0 + p < nf) step(buf[p]);
      buf[p] = issue();
    }
    if (++g == a.sync) {
      g = 0;
      __builtin_amdgcn_s_barrier();
    }
  }
}

size_t stream_lds(int SRC, int S, int KC, int hd, int Ck) {
  size_t lds = (size_t)S * (KC + 8) * 2;
  if (SRC != S_BUF) {
    const int Sk = SRC == S_SELF ? S : Ck;
    lds += (size_t)(S + 2 * Sk) * KC * 2 + (size_t)(KC / hd) * S * Sk * 4;
  }
  return lds;
}

template <int SRC, int EPI, int SPF, int NS, int WV>
int launch_stream_k(const SArgs& a, size_t lds, hipStream_t st) {
  // allow more than 64 KiB of dynamic LDS, once per device
  static unsigned long long attr_set = 0;
  int dev = 0;
  CFH_HIP(hipGetDevice(&dev));
  if (dev < 64 && !(attr_set & (1ull << dev))) {
    CFH_HIP(hipFuncSetAttribute((const void*)k_stream<SRC, EPI, SPF, NS, WV>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024));
    attr_set |= 1ull << dev;
  }
  const long long wgs = (long long)a.nex * a.ks * a.wg_per_kc * (EPI == E_PART16 ? std::max(a.nl, 1) : 1);
  if (a.conc > 1) {
    static int cus[64] = {};
    if (dev < 64 && !cus[dev]) CFH_HIP(hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev));
    if (dev < 64 && wgs * a.conc <= cus[dev]) lds = std::max(lds, CONC_LDS);
  }
  hipLaunchKernelGGL((k_stream<SRC, EPI, SPF, NS, WV>), dim3((unsigned)wgs), dim3(a.wpb * 64), lds, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// Operand loads per thread of an expert with S_max rows (16-byte vectors); more than 16 (or, for
// the cross attention, more than 4 q groups per thread) is not supported.
int stage_need(int SRC, const SArgs& a, int S_max) {
  const int nt = a.wpb * 64;
  auto up = [](int x, int y) { return (x + y - 1) / y; };
  const int KC = a.K / a.ks;
  if (SRC == S_BUF) return up(S_max * (KC / 8), nt);
  if (SRC == S_SELF) return up(3 * S_max * (KC / 8), nt);
  const int gj = up(S_max * (KC / 4), nt);
  return gj > 4 ? 1 << 20 : a.ks_in * gj + up(2 * a.Ck * (KC / 8), nt);
}

template <int SRC, int EPI, int SPF, int WV>
int launch_stream_ns(const SArgs& a, size_t lds, int need, hipStream_t st) {
  if (need <= 4) return launch_stream_k<SRC, EPI, SPF, 4, WV>(a, lds, st);
  if (need <= 8) return launch_stream_k<SRC, EPI, SPF, 8, WV>(a, lds, st);
  return launch_stream_k<SRC, EPI, SPF, 16, WV>(a, lds, st);
}

// Full-K units of 8-wave workgroups stream 160+ fragments per wave and want a deep prefetch;
// split-K units are short and many, and a shallower one keeps fewer requests queued at the HBM
// controllers; 16-wave workgroups already hold twice the waves per CU and take the shallower one
// (measured).  The operand slots (4, 8 or 16) cover every operand load of a thread.
// Operand slots of the kernel for a workgroup of wpb waves (the 16-wave kernels have 128 VGPRs).
int stage_slots(int wpb) { return wpb > 8 ? 8 : 16; }

int stream_check(int SRC, const SArgs& a, int S_max) {
  if (a.ks <= 0 || a.wpb <= 0 || a.tpw <= 0 || a.N % 16 || a.K % a.ks || (a.K / a.ks) % 32) return CFH_E_UNSUPPORTED;
  if (SRC != S_BUF && ((SRC == S_SELF ? S_max : a.Ck) > 16 || a.hd <= 0 || a.hd % 8 || (a.K / a.ks) % a.hd))
    return CFH_E_UNSUPPORTED;
  if ((a.N / 16) % (a.wpb * a.tpw) || a.wpb > SWMAX || stage_need(SRC, a, S_max) > stage_slots(a.wpb) ||
      stream_lds(SRC, S_max, a.K / a.ks, a.hd, a.Ck) > 150 * 1024)
    return CFH_E_UNSUPPORTED;
  return CFH_OK;
}

template <int SRC, int EPI>
int launch_stream(const SArgs& a0, int S_max, hipStream_t st) {
  SArgs a = a0;
  a.sync = STREAM_SYNC;
  if (stream_check(SRC, a, S_max)) return CFH_E_UNSUPPORTED;
  const size_t lds = stream_lds(SRC, S_max, a.K / a.ks, a.hd, a.Ck);
  const int need = stage_need(SRC, a, S_max);
  if (a.wpb > 8) {   // the 16-wave kernels have 128 VGPRs: at most 8 operand slots
    if (need <= 4) return launch_stream_k<SRC, EPI, PF_SPLIT, 4, 16>(a, lds, st);
    return launch_stream_k<SRC, EPI, PF_SPLIT, 8, 16>(a, lds, st);
  }
  if (a.ks == 1) return launch_stream_ns<SRC, EPI, PF_FULL, 8>(a, lds, need, st);
  return launch_stream_ns<SRC, EPI, PF_SPLIT, 8>(a, lds, need, st);
}

// ---------------------------------------------------------------------------- row kernels
// RES: the residual update of one row from the split-K partials of a sublayer, then the LayerNorm
// of the new row, a[r] = fp16(LN(fp16(x[r]))).  s = sum_kc P[kc][r] + bias:
//   RES_ADD32 : x += s                          (fp32 residual of the fused flow block)
//   RES_ADD16 : x = fp16(x + fp16(s))           (fp16 residual of torch modules: Linear, then add)
//   RES_POS16 : x = fp16(fp16(s) + pos[r])      (input Linear plus a position embedding row)
// One workgroup per (expert, row) of T threads (whole waves), NQ float4 column groups each; a row
// of d / 4 groups that does not fill T * NQ leaves the surplus lanes idle (their loads clamped
// into the row, their values masked).  The partial rows are loaded RB(NQ) at a time with every
// load of a batch in flight together.
enum ResMode { RES_ADD32 = 0, RES_ADD16 = 1, RES_POS16 = 2 };
constexpr int RQ = 4;             // max float4 groups per thread (d <= 16384 at 1024 threads)
// partial rows loaded per batch: as many as fit the registers of a launch bound of mt threads
// (mt 768: 168 VGPRs, mt 1024: 128)
constexpr int rb_for(int nq, int mt) {
  return mt <= 768 ? (nq <= 2 ? 8 : nq <= 4 ? 4 : nq <= 8 ? 2 : 1) : (nq <= 1 ? 8 : nq <= 2 ? 4 : nq <= 4 ? 2 : 1);
}

// NQ for a row of d columns: the smallest group count whose thread count (d / (4 NQ) rounded up to
// whole waves) is at most 1024 (0 if none), so the row's loads spread over as many lanes as
// possible; *threads receives that thread count.
int res_nq(int d, int* threads = nullptr) {
  const int nq = d / 4;
  if (d <= 0 || d % 4) return 0;
  for (int q = 1; q <= RQ; ++q) {
    const int t = ((nq + q - 1) / q + 63) / 64 * 64;
    if (t <= 1024) {
      if (threads) *threads = t;
      return q;
    }
  }
  return 0;
}

struct ResArgs {
  float* x[4];
  const float* P[4];
  const h16* bias[4];
  const h16* g[4];
  const h16* b[4];
  const h16* pos[4];   // RES_POS16: position rows [rows][d]
  h16* a[4];
  int rows[4];
  int nex, ks, d, mode;
  int pack;            // LN rows written in frag_index order (the folded cross attention's operand)
  int pos_period;      // RES_POS16: row r takes position row r % pos_period (sequences stacked; 0: r)
};

__device__ __forceinline__ float block_sum_rt(float v, float* red) {  // red[blockDim/64]
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  lds_barrier();   // (not __syncthreads: no wait for the row's global stores in flight)
  if (lane == 0) red[wave] = v;
  lds_barrier();
  float t = 0.f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += red[w];
  return t;
}

template <int NQ, int MT>
__device__ void res_row(const ResArgs& a, int e, int r) {
  __shared__ float red[16];
  const int RT = blockDim.x;
  const int d = a.d, nq = d / 4;
  const size_t pst = (size_t)a.rows[e] * d;
  float* xr = a.x[e] + (size_t)r * d;
  const float* Pr = a.P[e] + (size_t)r * d;
  const h16* pr = a.mode == RES_POS16 ? a.pos[e] + (size_t)(a.pos_period > 0 ? r % a.pos_period : r) * d : a.bias[e];
  // every load of the row is issued up front (the bias, gamma and beta too, so that the LayerNorm
  // does not pay a second memory round trip after the statistics); lanes past the row read its
  // last group
  float4 acc[NQ], xv[NQ];
  h16x4 bq[NQ], gq[NQ], btq[NQ], pq[NQ];
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int q = min((int)threadIdx.x + k * RT, nq - 1);
    xv[k] = *(const float4*)(xr + q * 4);
    acc[k] = *(const float4*)(Pr + q * 4);
    bq[k] = *(const h16x4*)(a.bias[e] + q * 4);
    gq[k] = *(const h16x4*)(a.g[e] + q * 4);
    btq[k] = *(const h16x4*)(a.b[e] + q * 4);
    pq[k] = *(const h16x4*)(pr + q * 4);
  }
  constexpr int RB = rb_for(NQ, MT);
  for (int kc = 1; kc < a.ks; kc += RB) {
    float4 t[RB][NQ];
#pragma unroll
    for (int u = 0; u < RB; ++u)
#pragma unroll
      for (int k = 0; k < NQ; ++k)
        t[u][k] = kc + u < a.ks ? *(const float4*)(Pr + (kc + u) * pst + min((int)threadIdx.x + k * RT, nq - 1) * 4)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < RB; ++u)
#pragma unroll
      for (int k = 0; k < NQ; ++k)
        if (kc + u < a.ks) {
          acc[k].x += t[u][k].x; acc[k].y += t[u][k].y; acc[k].z += t[u][k].z; acc[k].w += t[u][k].w;
        }
  }
  auto upd = [&](float x, float s, float b, float p) -> float {
    if (a.mode == RES_ADD32) return x + (s + b);
    if (a.mode == RES_ADD16) return r16(x + r16(s + b));
    return r16(r16(s + b) + p);
  };
  float4 vals[NQ];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int q = threadIdx.x + k * RT;
    float4 xn;
    xn.x = upd(xv[k].x, acc[k].x, (float)bq[k][0], (float)pq[k][0]);
    xn.y = upd(xv[k].y, acc[k].y, (float)bq[k][1], (float)pq[k][1]);
    xn.z = upd(xv[k].z, acc[k].z, (float)bq[k][2], (float)pq[k][2]);
    xn.w = upd(xv[k].w, acc[k].w, (float)bq[k][3], (float)pq[k][3]);
    if (q < nq) *(float4*)(xr + q * 4) = xn;
    vals[k] = q < nq ? r16x4(xn) : make_float4(0.f, 0.f, 0.f, 0.f);
    s += (vals[k].x + vals[k].y) + (vals[k].z + vals[k].w);
  }
  const float mean = block_sum_rt(s, red) / (float)d;
  float v = 0.f;
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const float a0 = vals[k].x - mean, a1 = vals[k].y - mean, a2 = vals[k].z - mean, a3 = vals[k].w - mean;
    if (threadIdx.x + k * RT < nq) v += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
  }
  const float rstd = 1.0f / sqrtf(block_sum_rt(v, red) / (float)d + LN_EPS);
  h16* out = a.a[e] + (size_t)r * d;
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int c = (threadIdx.x + k * RT) * 4;
    h16x4 o;
    o[0] = (h16)((vals[k].x - mean) * rstd * (float)gq[k][0] + (float)btq[k][0]);
    o[1] = (h16)((vals[k].y - mean) * rstd * (float)gq[k][1] + (float)btq[k][1]);
    o[2] = (h16)((vals[k].z - mean) * rstd * (float)gq[k][2] + (float)btq[k][2]);
    o[3] = (h16)((vals[k].w - mean) * rstd * (float)gq[k][3] + (float)btq[k][3]);
    if (c < d) *(h16x4*)(a.pack ? a.a[e] + frag_index(r, c, a.rows[e]) : out + c) = o;
  }
}

// MT = the launch bound: 768 threads (12 waves, up to 168 VGPRs) when the row fits, else 1024
// (128 VGPRs); the all-loads-up-front row needs more than 128 at NQ = 2.
template <int NQ, int MT>
__global__ void __launch_bounds__(MT) k_res(ResArgs a) {
  int e = 0, r = blockIdx.x;
  while (e + 1 < a.nex && r >= a.rows[e]) r -= a.rows[e++];
  res_row<NQ, MT>(a, e, r);
}

int launch_res(const ResArgs& a, hipStream_t st) {
  int total = 0;
  for (int e = 0; e < a.nex; ++e) total += a.rows[e];
  int threads = 0;
  const int NQ = res_nq(a.d, &threads);
  const bool small = threads <= 768;
  switch (NQ) {
#define CFH_RES(N) \
  case N:                                                                             \
    if (small) hipLaunchKernelGGL((k_res<N, 768>), dim3(total), dim3(threads), 0, st, a); \
    else hipLaunchKernelGGL((k_res<N, 1024>), dim3(total), dim3(threads), 0, st, a);      \
    break;
    CFH_RES(1) CFH_RES(2) CFH_RES(3) CFH_RES(4)
#undef CFH_RES
    default: return CFH_E_UNSUPPORTED;
  }
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// ---------------------------------------------------------------------------- host side
// Split-K factor of a streaming GEMV: the smallest divisor of the k-step count that leaves at
// least 8 k-steps per unit, keeps the A chunk within `lds_cap`, and gives >= `target` wave units;
// else the largest valid one.
int choose_ks(int nex, int tiles, int K, int S, int target, size_t lds_cap) {
  const int steps = K / 32;
  int best = -1;
  for (int ks = 1; ks <= steps; ++ks) {
    if (steps % ks || steps / ks < 8) continue;
    if ((size_t)S * (K / ks + 8) * 2 > lds_cap) continue;
    best = ks;
    if ((long long)nex * ks * tiles >= target) break;
  }
  return best;
}

// Waves per workgroup for a launch of nunits (expert, k-chunk) units of `tiles` column tiles: the
// most (at most maxw, a power of two dividing tiles) that still gives about one workgroup per CU
// (nunits * tiles / w >= 240); narrow widths take fewer waves so that the launch spans the chip.
// `vecs` (the operand's 8-half vectors, S rows x K-chunk / 8) raises the count again until every
// thread's operand loads fit its slots (16 up to 8 waves, 8 above).
int wpb_for_grid(int tiles, int nunits, int maxw, int vecs) {
  auto fits = [&](int w) { return (vecs + 64 * w - 1) / (64 * w) <= (w > 8 ? 8 : 16); };
  int best = 1;
  for (int w = 2; w <= maxw && tiles % w == 0 && (long long)nunits * tiles / w >= 240; w *= 2) best = w;
  while (!fits(best) && best * 2 <= maxw && tiles % (best * 2) == 0) best *= 2;
  return best;
}

int pick_wpb(int tiles, int tpw) {
  for (int w : {8, 4, 2, 1})
    if (tiles % (w * tpw) == 0) return w;
  return 1;
}

// Waves per workgroup (and, if tpw is given, tiles per wave: 1 or 2) that cut T tiles of each of U
// (expert, k-chunk) units into exactly one workgroup per CU of the 256, so the launch runs as one
// round; false (nothing changed) if no split of at most 16 waves does.
bool fit_grid(int T, int U, int* wpb, int* tpw) {
  constexpr int CUS = 256;
  if ((long long)T * U % CUS) return false;
  const int wt = (int)((long long)T * U / CUS);
  for (int tp : {2, 1}) {
    if ((tp == 2 && !tpw) || wt % tp || wt / tp > SWMAX || T % wt) continue;
    *wpb = wt / tp;
    if (tpw) *tpw = tp;
    return true;
  }
  return false;
}

}  // namespace
