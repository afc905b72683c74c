// The chain-flow velocity net + Euler integrator on MI355X: TreeFlowDrafter.predict_hidden.
//
// Reference semantics (cf/ = src/chain_flow/): init_latents cf/drafters/tree_flow.py:150-161,
// integrate :229-235, flow_velocity/_chunk_args :163-190, HiddenKVFlowExpert.pre_blocks /
// post_blocks cf/drafters/chunked_flow.py:333-384, HiddenKVFlowBlock.forward :185-202; fused-kernel
// numerics cf/csrc/fused_block.cu:280-325, 452-668, 674-722 (fp32 residual, fp16-parked LayerNorm
// rows, fp16 q/k/v, attention and GELU outputs, cross K/V hoisted once per draft).
//
// Execution plan.  One launch sequence per draft on the caller's stream; every launch covers both
// chunk experts (they are independent within an Euler step), so each weight-streaming launch moves
// the weights of two experts.  Work that needs a whole row sits in a small row kernel between two
// streaming kernels; there is no cross-workgroup synchronisation inside any kernel (no fences, no
// atomics, no spin-waits), so results are deterministic.  On MI355X a kernel boundary costs about
// nothing on the stream, while a fenced grid barrier across the 8 XCDs costs ~12 us, which is why
// this is a kernel pipeline and not one persistent launch.
//
//   per draft : TAU  time_mlp(tau_s) for all E steps     (GEMV + reduce)
//               ROWS init_latents(ctx), step-0 rows x, a = LN_self(x) of block 0
//               KV   cross K/V of every block             (GEMV + reduce)
//   per Euler step, per block l (both experts in every launch):
//     QKV   stream  A = a (LN_self rows)          epilogue q,k,v = fp16(acc + b)      full-K tiles
//     O     stream  A = causal self attention of head h, computed while staging    split-K by head
//     RES   row     x += sum_h P + b_o ; a = LN_cross(fp16(x))
//     QC    stream  A = a                         fp32 partials                     split-K
//     OC    stream  A = cross attention of head h (q reduced from the QC partials, hoisted K/V)
//     RES   row     x += sum_h P + b_oc ; a = LN_ffn(fp16(x))
//     W1    stream  A = a                         epilogue g = fp16(gelu(acc + b1))  full-K tiles
//     W2    stream  A = g                         fp32 partials                     split-K
//     RES   row     x += sum P + b2 ; a = LN_self of block l+1 (out_norm after the last block)
//   OUT   stream  A = out_norm rows of the current chunk                           split-K
//   ROWS  row     v = fp16(sum P + b_out); z = fp16(z + fp16(dt v)); next step's rows and LN_self
//
// Streaming kernel: a wave owns TPW consecutive 16-column tiles of one (expert, k-chunk); it
// streams their packed fragments (1 KiB per wave per k-step, contiguous per tile, non-temporal)
// with PF fragment loads in flight, issued before the A operand is staged, and multiplies each
// against the A rows held in LDS with v_mfma_f32_16x16x32_f16.
#include <stdio.h>

#include <algorithm>

#include "cfh_kernels.h"

namespace {

constexpr int SWMAX = 16;         // max waves per streaming workgroup
constexpr int PF_FULL = 16;       // fragment loads in flight per wave: full-K kernels
constexpr int PF_SPLIT = 8;       //                                   split-K kernels
constexpr int STREAM_SYNC = 4;    // fragment groups between workgroup barriers in the stream (measured: 4 best of 0-4)

enum SrcKind { S_BUF = 0, S_SELF = 1, S_CROSS = 2 };
enum EpiKind { E_PART = 0, E_BIAS16 = 1, E_GELU16 = 2 };

struct SEx {
  const h16x8* w;      // packed weights: fragment (tile t, k-step s) at ((t * K/32) + s) * 64
  const h16* a;        // S_BUF: rows [S][lda] | S_SELF: q,k,v rows [S][3d] | S_CROSS: K/V [2][Ck][d]
  int lda;
  const float* pin;    // S_CROSS: cross-q partials [ks_in][S][d]
  const h16* bin;      // S_CROSS: cross-q bias (in_proj_bias[0:d])
  const h16* bias;     // E_BIAS16 / E_GELU16 bias [N]
  void* out;           // E_PART: float [ks][S][N]; otherwise h16 [S][N]
  int S;               // activation rows (<= 16)
};

struct SArgs {
  SEx ex[4];
  int nex, N, K, ks, wpb, tpw, wg_per_kc;
  int d, hd, ks_in, Ck;
  int sync;            // fragment groups between workgroup barriers in the stream (0: none)
};

// Attention of head h for the S rows of one expert from q, k, v already in LDS (sq [S][hd], sk and
// sv [Sk][hd], Sk <= 16), written as fp16 into As [S][lda].  Causal mask = triu(-inf, 1)
// (cf/drafters/chunked_flow.py:273-275); scores and the weighted sum in fp32 on fp16 q/k/v, output
// rounded to fp16.
// One wave per query row: lane group j (LP lanes) holds key j, so the dot products, the row max,
// exp and sum stay in registers (DPP reductions); every LDS read of a phase is issued before the
// first is used.  (A wave per (i, j) pair with a serial softmax thread per row spent 2-4 us here,
// almost all of it in dependent LDS round trips.)
__device__ void attend(int S, int Sk, int hd, bool causal, const h16* sq, const h16* sk, const h16* sv,
                       float* P, h16* As, int lda) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const float scale = 1.0f / sqrtf((float)hd);
  const bool l8 = Sk <= 8;                 // 8 lanes per key (else 4)
  const int j = l8 ? lane >> 3 : lane >> 2, sub = l8 ? lane & 7 : lane & 3;
  const int step = l8 ? 64 : 32;           // halves between a lane's 8-half chunks
  const int jr = min(j, Sk - 1);           // lanes of keys >= Sk read a valid row, result masked
  for (int i = wave; i < S; i += nw) {
    const h16* qr = sq + i * hd + sub * 8;
    const h16* kr = sk + jr * hd + sub * 8;
    float part = 0.f;
    for (int c = 0; c < hd; c += step) {
      const h16x8 qa = *(const h16x8*)(qr + c);
      const h16x8 kb = *(const h16x8*)(kr + c);
#pragma unroll
      for (int t = 0; t < 8; ++t) part += (float)qa[t] * (float)kb[t];
    }
    part += dpp_f32<DPP_XOR1>(part);
    part += dpp_f32<DPP_XOR2>(part);
    if (l8) part += dpp_f32<DPP_HMIRROR>(part);
    const bool valid = j < Sk && !(causal && j > i);
    const float sc = valid ? part * scale : -INFINITY;
    const float m = wave_max(sc);
    const float e = valid ? expf(sc - m) : 0.f;
    const float inv = 1.0f / wave_sum(sub == 0 ? e : 0.f);
    if (sub == 0 && j < Sk) P[i * Sk + j] = e * inv;
  }
  lds_barrier();
  const int nv = hd / 8;
  for (int idx = threadIdx.x; idx < S * nv; idx += blockDim.x) {
    const int i = idx / nv, c = (idx - i * nv) * 8;
    float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j0 = 0; j0 < Sk; j0 += 8) {   // 8 keys at a time; keys past Sk: a valid row, weight 0
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int jc = min(j0 + jj, Sk - 1);
        const float p = j0 + jj < Sk ? P[i * Sk + jc] : 0.f;
        const h16x8 vb = *(const h16x8*)(sv + jc * hd + c);
#pragma unroll
        for (int t = 0; t < 8; ++t) o[t] += p * (float)vb[t];
      }
    }
    h16x8 ov;
#pragma unroll
    for (int t = 0; t < 8; ++t) ov[t] = (h16)o[t];
    *(h16x8*)(As + i * lda + c) = ov;
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
//   S_SELF : vectors of q | k | v of head h (each [S][hd]) -> consecutive LDS blocks sq, sk, sv
//   S_CROSS: the ks_in fp32 partials of each 4-column q group g = t + j * nt the thread owns
//            (slot q * gj + j; summed in the order q = 0, 1, ...) and then the vectors of the
//            hoisted context K and V rows of head h
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
  __device__ __forceinline__ static const h16x8* self_src(const SArgs& a, const SEx& ex, int h, int nv, int idx) {
    const int part = idx / (ex.S * nv);
    const int r = idx - part * ex.S * nv;
    const int i = r / nv, c = (r - i * nv) * 8;
    return (const h16x8*)(ex.a + (size_t)i * 3 * a.d + part * a.d + h * a.hd + c);
  }
  __device__ __forceinline__ static const h16x8* kv_src(const SArgs& a, const SEx& ex, int h, int nv, int idx) {
    const int j = idx / nv, c = (idx - j * nv) * 8;   // j < 2 Ck: K rows then V rows
    return (const h16x8*)(ex.a + (size_t)j * a.d + h * a.hd + c);
  }
  __device__ __forceinline__ static const h16x8* q_src(const SArgs& a, const SEx& ex, int h, int g, int q) {
    const int nq = a.hd / 4;
    const int i = g / nq, c = (g - i * nq) * 4;
    return (const h16x8*)(ex.pin + (size_t)q * ex.S * a.d + (size_t)i * a.d + h * a.hd + c);
  }

  __device__ __forceinline__ void load(const SArgs& a, const SEx& ex, int kc, int KC) {
    const int t = threadIdx.x, nt = blockDim.x;
    if constexpr (SRC == S_BUF) {
      const int nv = KC / 8, total = ex.S * nv;
#pragma unroll
      for (int u = 0; u < NS; ++u) st[u] = *buf_src(ex, kc, KC, nv, min(u * nt + t, total - 1));
    } else if constexpr (SRC == S_SELF) {
      const int nv = a.hd / 8, total = 3 * ex.S * nv;
#pragma unroll
      for (int u = 0; u < NS; ++u) st[u] = *self_src(a, ex, kc, nv, min(u * nt + t, total - 1));
    } else {
      const int G = ex.S * (a.hd / 4), nv = a.hd / 8, nkv = 2 * a.Ck * nv;
      gj = (G + nt - 1) / nt;
      nqs = a.ks_in * gj;
      const int nq = a.hd / 4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int g = min(t + j * nt, G - 1);
        qb[j] = *(const uint2*)(ex.bin + kc * a.hd + (g - (g / nq) * nq) * 4);
      }
#pragma unroll
      for (int u = 0; u < NS; ++u) {
        if (u < nqs) {
          const int q = u / gj, j = u - q * gj;
          st[u] = *q_src(a, ex, kc, min(t + j * nt, G - 1), q);
        } else {
          st[u] = *kv_src(a, ex, kc, nv, min((u - nqs) * nt + t, nkv - 1));
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
      const int S = ex.S, hd = a.hd, nv = hd / 8;
      const int Sk = SRC == S_SELF ? S : a.Ck;
      h16* sq = As + (size_t)S * lda;
      h16* sk = sq + (size_t)S * hd;
      h16* sv = sk + (size_t)Sk * hd;
      float* P = (float*)(sv + (size_t)Sk * hd);   // [S][Sk]
      if constexpr (SRC == S_SELF) {
        const int total = 3 * S * nv;
#pragma unroll
        for (int u = 0; u < NS; ++u) *(h16x8*)(sq + (size_t)min(u * nt + t, total - 1) * 8) = st[u];
      } else {
        const int nq = hd / 4, G = S * nq, nkv = 2 * Sk * nv;
        // q = fp16(sum of the cross-q partials + bias) for the 4-column group g
        auto put_q = [&](int g, float4 s4, uint2 bw) {
          const int i = g / nq, c = (g - i * nq) * 4;
          const h16x4 bb = __builtin_bit_cast(h16x4, bw);
          h16* dst = sq + i * hd + c;
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
      attend(S, Sk, hd, SRC == S_SELF, sq, sk, sv, P, As, lda);
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
  const int e = b / per_ex;
  b -= e * per_ex;
  const int kc = b / a.wg_per_kc;
  const int tg = b - kc * a.wg_per_kc;
  const SEx& ex = a.ex[e];
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
  if constexpr (EPI != E_PART) bias0 = (float)ex.bias[t0 * 16 + (lane & 15)];
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
          } else {
            float bv;
            if (ct == 0) bv = bias0;
            else bv = (float)ex.bias[n];
            if constexpr (EPI == E_BIAS16) ((h16*)ex.out)[(size_t)r * a.N + n] = (h16)(acc[q] + bv);
            else ((h16*)ex.out)[(size_t)r * a.N + n] = (h16)gelu_erf(acc[q] + bv);
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
    lds += (size_t)(S + 2 * Sk) * hd * 2 + (size_t)S * Sk * 4;
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
  const long long wgs = (long long)a.nex * a.ks * a.wg_per_kc;
  hipLaunchKernelGGL((k_stream<SRC, EPI, SPF, NS, WV>), dim3((unsigned)wgs), dim3(a.wpb * 64), lds, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// Operand loads per thread of an expert with S_max rows (16-byte vectors); more than 16 (or, for
// the cross attention, more than 4 q groups per thread) is not supported.
int stage_need(int SRC, const SArgs& a, int S_max) {
  const int nt = a.wpb * 64;
  auto up = [](int x, int y) { return (x + y - 1) / y; };
  if (SRC == S_BUF) return up(S_max * (a.K / a.ks / 8), nt);
  if (SRC == S_SELF) return up(3 * S_max * (a.hd / 8), nt);
  const int gj = up(S_max * (a.hd / 4), nt);
  return gj > 4 ? 1 << 20 : a.ks_in * gj + up(2 * a.Ck * (a.hd / 8), nt);
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
  if (SRC != S_BUF && ((SRC == S_SELF ? S_max : a.Ck) > 16 || a.hd % 64)) return CFH_E_UNSUPPORTED;
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
// RES: x[r] += sum_kc P[kc][r] + bias; a[r] = fp16(LN(fp16(x[r]))).  One workgroup per (expert,
// row) of d / (4 NQ) threads, NQ float4 column groups each; the partial rows are loaded RB(NQ) at a
// time with every load of a batch in flight together.
constexpr int RQ = 16;            // max float4 groups per thread (d <= 16384)
// partial rows loaded per batch: as many as fit the registers of a launch bound of mt threads
// (mt 768: 168 VGPRs, mt 1024: 128)
constexpr int rb_for(int nq, int mt) {
  return mt <= 768 ? (nq <= 2 ? 8 : nq <= 4 ? 4 : nq <= 8 ? 2 : 1) : (nq <= 1 ? 8 : nq <= 2 ? 4 : nq <= 4 ? 2 : 1);
}

// NQ for a row of d columns: the smallest group count giving a whole number of waves and at most
// 1024 threads (0 if none), so the row's loads spread over as many lanes as possible.
int res_nq(int d) {
  const int nq = d / 4;
  for (int q = 1; q <= RQ; ++q)
    if (nq % q == 0 && (nq / q) % 64 == 0 && nq / q <= 1024) return q;
  return 0;
}

struct ResArgs {
  float* x[4];
  const float* P[4];
  const h16* bias[4];
  const h16* g[4];
  const h16* b[4];
  h16* a[4];
  int rows[4];
  int nex, ks, d;
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
  const int d = a.d;
  const size_t pst = (size_t)a.rows[e] * d;
  float* xr = a.x[e] + (size_t)r * d;
  const float* Pr = a.P[e] + (size_t)r * d;
  // every load of the row is issued up front (the bias, gamma and beta too, so that the LayerNorm
  // does not pay a second memory round trip after the statistics)
  float4 acc[NQ], xv[NQ];
  h16x4 bq[NQ], gq[NQ], btq[NQ];
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int q = threadIdx.x + k * RT;
    xv[k] = *(const float4*)(xr + q * 4);
    acc[k] = *(const float4*)(Pr + q * 4);
    bq[k] = *(const h16x4*)(a.bias[e] + q * 4);
    gq[k] = *(const h16x4*)(a.g[e] + q * 4);
    btq[k] = *(const h16x4*)(a.b[e] + q * 4);
  }
  constexpr int RB = rb_for(NQ, MT);
  for (int kc = 1; kc < a.ks; kc += RB) {
    float4 t[RB][NQ];
#pragma unroll
    for (int u = 0; u < RB; ++u)
#pragma unroll
      for (int k = 0; k < NQ; ++k)
        t[u][k] = kc + u < a.ks ? *(const float4*)(Pr + (kc + u) * pst + (threadIdx.x + k * RT) * 4)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < RB; ++u)
#pragma unroll
      for (int k = 0; k < NQ; ++k)
        if (kc + u < a.ks) {
          acc[k].x += t[u][k].x; acc[k].y += t[u][k].y; acc[k].z += t[u][k].z; acc[k].w += t[u][k].w;
        }
  }
  float4 vals[NQ];
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const int q = threadIdx.x + k * RT;
    float4 xn;
    xn.x = xv[k].x + (acc[k].x + (float)bq[k][0]);
    xn.y = xv[k].y + (acc[k].y + (float)bq[k][1]);
    xn.z = xv[k].z + (acc[k].z + (float)bq[k][2]);
    xn.w = xv[k].w + (acc[k].w + (float)bq[k][3]);
    *(float4*)(xr + q * 4) = xn;
    vals[k] = r16x4(xn);
    s += (vals[k].x + vals[k].y) + (vals[k].z + vals[k].w);
  }
  const float mean = block_sum_rt(s, red) / (float)d;
  float v = 0.f;
#pragma unroll
  for (int k = 0; k < NQ; ++k) {
    const float a0 = vals[k].x - mean, a1 = vals[k].y - mean, a2 = vals[k].z - mean, a3 = vals[k].w - mean;
    v += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
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
    *(h16x4*)(out + c) = o;
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
  const int NQ = res_nq(a.d);
  const int threads = NQ ? a.d / 4 / NQ : 0;
  const bool small = threads <= 768;
  switch (NQ) {
#define CFH_RES(N) \
  case N:                                                                             \
    if (small) hipLaunchKernelGGL((k_res<N, 768>), dim3(total), dim3(threads), 0, st, a); \
    else hipLaunchKernelGGL((k_res<N, 1024>), dim3(total), dim3(threads), 0, st, a);      \
    break;
    CFH_RES(1) CFH_RES(2) CFH_RES(3) CFH_RES(4) CFH_RES(5) CFH_RES(6) CFH_RES(7) CFH_RES(8)
    CFH_RES(9) CFH_RES(10) CFH_RES(11) CFH_RES(12) CFH_RES(13) CFH_RES(14) CFH_RES(15) CFH_RES(16)
#undef CFH_RES
    default: return CFH_E_UNSUPPORTED;
  }
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// ROWS: one workgroup per z row r.
//   init  : z[r] = init_latents(ctx)[r] (delta mode, fp16 arithmetic); context row moments
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
    for (int kc = 1; kc < a.ks; kc += 2) {
      float4 t[2][ROWQ];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int k = 0; k < ROWQ; ++k) {
          const int q = threadIdx.x + k * blockDim.x;
          t[u][k] = (q < nq && kc + u < a.ks) ? *(const float4*)(Pr + (kc + u) * pst + q * 4)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int k = 0; k < ROWQ; ++k)
          if (kc + u < a.ks) { acc[k].x += t[u][k].x; acc[k].y += t[u][k].y; acc[k].z += t[u][k].z; acc[k].w += t[u][k].w; }
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

struct Plan {
  int d, fd, CS, E, NL, C, KD, H, hd, nch, Smax;
  int ks_qc, ks_w2, ks_out, ks_kv, ks_tau;
  int wpb_qc, wpb_w2, wpb_out, tpw_att, wpb_att, wpb_full, wpb_w1;
  int pks;            // partial slots per expert
  bool ok;
};

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

Plan make_plan(const cfh_flow_dims* dm) {
  Plan p = {};
  p.d = dm->d; p.fd = dm->ffn_mult * dm->d; p.CS = dm->chunk_size; p.E = dm->flow_steps;
  p.NL = dm->layers; p.C = dm->ctx_rows; p.KD = dm->draft_length; p.H = dm->heads; p.hd = p.d / p.H;
  p.nch = p.KD / p.CS;
  p.Smax = p.KD;
  const int tiles_d = p.d / 16;
  const size_t cap = 96 * 1024;
  p.ks_qc = choose_ks(p.nch, tiles_d, p.d, p.Smax, 2048, cap);
  // W2: one d-wide k-chunk per ffn slice (ks = ffn_mult) in 16-wave workgroups, so that W1 and W2
  // both run as one round of ~240 workgroups at one workgroup per CU; else split-K by wave count
  const bool w2_wide = tiles_d % 16 == 0 && stream_lds(S_BUF, p.Smax, p.d, p.hd, p.C) <= 150 * 1024;
  p.ks_w2 = w2_wide ? dm->ffn_mult : choose_ks(p.nch, tiles_d, p.fd, p.Smax, 4096, cap);
  p.ks_out = choose_ks(p.nch, tiles_d, p.d, p.CS, 2048, cap);
  p.ks_kv = ksplit_for(p.nch * p.NL, 2 * p.d / 16, p.d, p.C);
  p.ks_tau = ksplit_for(p.nch, p.d / 16, p.d, p.E);
  p.wpb_qc = std::min(4, pick_wpb(tiles_d, 1));
  p.wpb_w2 = w2_wide ? 16 : std::min(4, pick_wpb(tiles_d, 1));
  p.wpb_out = pick_wpb(tiles_d, 1);
  p.tpw_att = (tiles_d % 16 == 0) ? 2 : 1;
  p.wpb_att = pick_wpb(tiles_d, p.tpw_att);
  fit_grid(tiles_d, p.nch * p.H, &p.wpb_att, &p.tpw_att);
  p.wpb_full = 8;
  p.wpb_w1 = (p.fd / 16) % 16 == 0 ? 16 : 8;
  // the cross attention holds every q partial of its groups in registers: fewer QC splits if needed
  for (int ks = p.ks_qc; ks > 1; --ks) {
    SArgs a = {};
    a.N = p.d; a.K = p.d; a.ks = p.H; a.wpb = p.wpb_att; a.tpw = p.tpw_att; a.hd = p.hd; a.ks_in = ks; a.Ck = p.C;
    if ((p.d / 32) % ks || stage_need(S_CROSS, a, p.Smax) > stage_slots(a.wpb)) continue;
    p.ks_qc = ks;
    break;
  }
  fit_grid(tiles_d, p.nch * p.ks_qc, &p.wpb_qc, nullptr);
  fit_grid(tiles_d, p.nch * p.ks_out, &p.wpb_out, nullptr);
  p.pks = std::max(std::max(p.H, p.ks_w2), p.ks_out);
  p.ok = p.ks_qc > 0 && p.ks_qc <= 8 && p.ks_w2 > 0 && p.ks_out > 0 && p.hd % 32 == 0 && res_nq(p.d) > 0;
  if (!p.ok) return p;
  // every streaming launch of a draft, as block_pass and the OUT step issue them
  auto sa = [&](int N, int K, int ks, int wpb, int tpw) {
    SArgs a = {};
    a.nex = p.nch; a.N = N; a.K = K; a.ks = ks; a.wpb = wpb; a.tpw = tpw; a.d = p.d; a.hd = p.hd;
    a.ks_in = p.ks_qc; a.Ck = p.C;
    return a;
  };
  p.ok = !stream_check(S_BUF, sa(3 * p.d, p.d, 1, p.wpb_full, 1), p.Smax) &&
         !stream_check(S_SELF, sa(p.d, p.d, p.H, p.wpb_att, p.tpw_att), p.Smax) &&
         !stream_check(S_BUF, sa(p.d, p.d, p.ks_qc, p.wpb_qc, 1), p.Smax) &&
         !stream_check(S_CROSS, sa(p.d, p.d, p.H, p.wpb_att, p.tpw_att), p.Smax) &&
         !stream_check(S_BUF, sa(p.fd, p.d, 1, p.wpb_w1, 1), p.Smax) &&
         !stream_check(S_BUF, sa(p.d, p.fd, p.ks_w2, p.wpb_w2, 1), p.Smax) &&
         !stream_check(S_BUF, sa(p.d, p.d, p.ks_out, p.wpb_out, 1), p.CS);
  return p;
}

struct WS {
  float* z;
  float* x[4];
  h16* abuf[4];
  h16* qkv[4];
  h16* g[4];
  float* P[4];        // partials of the split-K kernels (O, OC, W2, OUT)
  float* Pq[4];       // cross-q partials (QC), read by OC
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
    w.qkv[c] = (h16*)take(S * 3 * d * 2);
    w.g[c] = (h16*)take(S * fd * 2);
    w.P[c] = (float*)take((size_t)p.pks * S * d * 4);
    w.Pq[c] = (float*)take((size_t)p.ks_qc * S * d * 4);
    w.tau[c] = (h16*)take((size_t)p.E * d * 2);
    w.kvc[c] = (h16*)take((size_t)p.NL * 2 * p.C * d * 2);
  }
  w.Pkv = (float*)take((size_t)p.nch * p.NL * p.ks_kv * p.C * 2 * d * 4);
  w.Ptau = (float*)take((size_t)p.nch * p.ks_tau * p.E * d * 4);
  w.ctx_mom = (float*)take((size_t)p.C * 2 * 4);
  w.total = off;
  return w;
}

// The nine launches of block l (both experts in each).
int block_pass(const Plan& p, const cfh::ExpertLayout& L, const WS& w, const void* const* experts, int l,
               hipStream_t st) {
  const int d = p.d, fd = p.fd, NL = p.NL, nch = p.nch;
  auto PTR = [&](int c, size_t off) { return (const char*)experts[c] + off; };
  const size_t B = L.blk0 + (size_t)l * L.blkstride;
  auto S_of = [&](int c) { return (c + 1) * p.CS; };
  int rc;
  // QKV: q, k, v = fp16(LN_self(x) W_in^T + b_in), full-K tiles
  {
    SArgs a = {};
    a.nex = nch; a.N = 3 * d; a.K = d; a.ks = 1; a.wpb = p.wpb_full; a.tpw = 1; a.d = d; a.hd = p.hd;
    a.wg_per_kc = (3 * d / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.qkv); x.a = w.abuf[c]; x.lda = d; x.bias = (const h16*)PTR(c, B + L.qkv_b);
      x.out = w.qkv[c]; x.S = S_of(c);
    }
    if ((rc = launch_stream<S_BUF, E_BIAS16>(a, p.Smax, st))) return rc;
  }
  // O: causal self attention per head, staged, then out_proj split-K by head
  {
    SArgs a = {};
    a.nex = nch; a.N = d; a.K = d; a.ks = p.H; a.wpb = p.wpb_att; a.tpw = p.tpw_att; a.d = d; a.hd = p.hd;
    a.wg_per_kc = (d / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.o); x.a = w.qkv[c]; x.out = w.P[c]; x.S = S_of(c);
    }
    if ((rc = launch_stream<S_SELF, E_PART>(a, p.Smax, st))) return rc;
  }
  ResArgs r = {};
  r.nex = nch; r.d = d;
  for (int c = 0; c < nch; ++c) { r.x[c] = w.x[c]; r.P[c] = w.P[c]; r.a[c] = w.abuf[c]; r.rows[c] = S_of(c); }
  // residual + LN_cross
  r.ks = p.H;
  for (int c = 0; c < nch; ++c) {
    r.bias[c] = (const h16*)PTR(c, B + L.o_b);
    r.g[c] = (const h16*)PTR(c, B + L.xn_w); r.b[c] = (const h16*)PTR(c, B + L.xn_b);
  }
  if ((rc = launch_res(r, st))) return rc;
  // QC: cross-attention query projection, split-K partials
  {
    SArgs a = {};
    a.nex = nch; a.N = d; a.K = d; a.ks = p.ks_qc; a.wpb = p.wpb_qc; a.tpw = 1; a.d = d; a.hd = p.hd;
    a.wg_per_kc = (d / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.qc); x.a = w.abuf[c]; x.lda = d; x.out = w.Pq[c]; x.S = S_of(c);
    }
    if ((rc = launch_stream<S_BUF, E_PART>(a, p.Smax, st))) return rc;
  }
  // OC: cross attention per head over the hoisted context K/V, staged, then out_proj split-K by head
  {
    SArgs a = {};
    a.nex = nch; a.N = d; a.K = d; a.ks = p.H; a.wpb = p.wpb_att; a.tpw = p.tpw_att; a.d = d; a.hd = p.hd;
    a.ks_in = p.ks_qc; a.Ck = p.C;
    a.wg_per_kc = (d / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.oc); x.a = w.kvc[c] + (size_t)l * 2 * p.C * d; x.pin = w.Pq[c];
      x.bin = (const h16*)PTR(c, B + L.qc_b); x.out = w.P[c]; x.S = S_of(c);
    }
    if ((rc = launch_stream<S_CROSS, E_PART>(a, p.Smax, st))) return rc;
  }
  // residual + LN_ffn
  for (int c = 0; c < nch; ++c) {
    r.bias[c] = (const h16*)PTR(c, B + L.oc_b);
    r.g[c] = (const h16*)PTR(c, B + L.fn_w); r.b[c] = (const h16*)PTR(c, B + L.fn_b);
  }
  if ((rc = launch_res(r, st))) return rc;
  // W1: g = fp16(gelu(LN_ffn(x) W1^T + b1)), full-K tiles
  {
    SArgs a = {};
    a.nex = nch; a.N = fd; a.K = d; a.ks = 1; a.wpb = p.wpb_w1; a.tpw = 1; a.d = d; a.hd = p.hd;
    a.wg_per_kc = (fd / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.w1); x.a = w.abuf[c]; x.lda = d; x.bias = (const h16*)PTR(c, B + L.w1_b);
      x.out = w.g[c]; x.S = S_of(c);
    }
    if ((rc = launch_stream<S_BUF, E_GELU16>(a, p.Smax, st))) return rc;
  }
  // W2: split-K partials
  {
    SArgs a = {};
    a.nex = nch; a.N = d; a.K = fd; a.ks = p.ks_w2; a.wpb = p.wpb_w2; a.tpw = 1; a.d = d; a.hd = p.hd;
    a.wg_per_kc = (d / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.w2); x.a = w.g[c]; x.lda = fd; x.out = w.P[c]; x.S = S_of(c);
    }
    if ((rc = launch_stream<S_BUF, E_PART>(a, p.Smax, st))) return rc;
  }
  // residual + LayerNorm of the next block (out_norm after the last block)
  r.ks = p.ks_w2;
  for (int c = 0; c < nch; ++c) {
    r.bias[c] = (const h16*)PTR(c, B + L.w2_b);
    if (l + 1 < NL) {
      const size_t Bn = L.blk0 + (size_t)(l + 1) * L.blkstride;
      r.g[c] = (const h16*)PTR(c, Bn + L.sn_w); r.b[c] = (const h16*)PTR(c, Bn + L.sn_b);
    } else {
      r.g[c] = (const h16*)PTR(c, L.on_w); r.b[c] = (const h16*)PTR(c, L.on_b);
    }
  }
  return launch_res(r, st);
}

}  // namespace

extern "C" {

int cfh_caps(const cfh_flow_dims* dims, int batch, int64_t* ws_bytes) {
  if (!cfh::flow_dims_ok(dims) || batch < 1) return CFH_E_UNSUPPORTED;
  if (dims->d > ROWT * ROWE || dims->draft_length > MAXR) return CFH_E_UNSUPPORTED;
  const Plan p = make_plan(dims);
  if (!p.ok) return CFH_E_UNSUPPORTED;
  const WS w = carve(p, nullptr);
  if (ws_bytes) *ws_bytes = (int64_t)w.total;
  return CFH_OK;
}

int cfh_flow_integrate(const cfh_flow_dims* dm, const void* const* experts, const void* ctx, void* z_out,
                       void* ws_ptr, int batch, void* stream) {
  if (!cfh::flow_dims_ok(dm) || dm->d > ROWT * ROWE || dm->draft_length > MAXR) return CFH_E_UNSUPPORTED;
  if (!experts || !ctx || !z_out || !ws_ptr || batch < 1) return CFH_E_INVALID;
  const Plan p = make_plan(dm);
  if (!p.ok) return CFH_E_UNSUPPORTED;
  for (int c = 0; c < p.nch; ++c)
    if (!experts[c]) return CFH_E_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const cfh::ExpertLayout L = cfh::expert_layout(dm);
  const WS w = carve(p, (char*)ws_ptr);
  const int d = p.d, CS = p.CS, E = p.E, NL = p.NL, C = p.C, KD = p.KD, nch = p.nch;
  int rc = CFH_OK;
  auto PTR = [&](int c, size_t off) { return (const char*)experts[c] + off; };
  auto BLK = [&](int l) { return L.blk0 + (size_t)l * L.blkstride; };

  for (int b = 0; b < batch; ++b) {
    const h16* ctx_b = (const h16*)ctx + (size_t)b * C * d;
    h16* zo_b = (h16*)z_out + (size_t)b * KD * d;

    // ---- per draft: time embeddings of every step
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
      r.ctx = ctx_b; r.ctx_mom = w.ctx_mom; r.z = w.z; r.z_out = zo_b; r.euler = 0; r.last = 0; r.d = d; r.C = C;
      r.CS = CS; r.nch = nch;
      for (int c = 0; c < nch; ++c) {
        r.x[c] = w.x[c]; r.pos[c] = (const h16*)PTR(c, L.pos); r.tau[c] = w.tau[c];
        r.g[c] = (const h16*)PTR(c, BLK(0) + L.sn_w); r.b[c] = (const h16*)PTR(c, BLK(0) + L.sn_b);
        r.a[c] = w.abuf[c];
      }
      hipLaunchKernelGGL(k_rows, dim3(KD), dim3(ROWT), 0, st, r);
      CFH_LAUNCH_CHECK();
    }
    // ---- cross K/V of every block (once per draft)
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
      for (int l = 0; l < NL; ++l)
        if ((rc = block_pass(p, L, w, experts, l, st))) return rc;
      // OUT: out_proj on the out_norm rows of each expert's current chunk
      {
        SArgs a = {};
        a.nex = nch; a.N = d; a.K = d; a.ks = p.ks_out; a.wpb = p.wpb_out; a.tpw = 1; a.d = d; a.hd = p.hd;
        a.wg_per_kc = (d / 16) / (a.wpb * a.tpw);
        for (int c = 0; c < nch; ++c) {
          SEx& x = a.ex[c];
          x.w = (const h16x8*)PTR(c, L.out); x.a = w.abuf[c] + (size_t)c * CS * d; x.lda = d; x.out = w.P[c];
          x.S = CS;
        }
        if ((rc = launch_stream<S_BUF, E_PART>(a, CS, st))) return rc;
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
