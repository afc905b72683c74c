// Wide request groups of the flow: many drafts share every weight stream.
//
// A batch of drafts is run in groups of up to 16 requests (128 activation rows for the second
// chunk expert at draft_length 8) whose rows all multiply each packed weight fragment as it
// streams past, so a group costs about one draft's weight traffic instead of one per two drafts.
// The narrow streaming kernel (cfh_stream.h) stages its whole K chunk once and holds at most 16
// rows; here the activation rows are staged in K chunks of WCH columns through two LDS buffers,
// refilled while the weights stream:
//
//   chunk c:  issue the loads of chunk c+1's rows into registers (they return after the weight
//             fragments already in flight, which the multiplies need first anyway)
//             multiply the chunk's WCH/32 k-steps of fragments, each against every 16-row group
//             of the rows in LDS
//             place chunk c+1's rows in the other buffer, one LDS barrier
//
// A wave owns WT adjacent 16-column tiles of one (expert, k-split) unit and keeps one accumulator
// per (tile, 16-row group).  Self attention, which the narrow kernel computes while staging, runs as its own
// small kernel per (request, head), and the context rows' LayerNorm of every block is computed
// once per draft into rows the cross K/V stream reads.
#pragma once
#include <algorithm>

#include "cfh_stream.h"

namespace {

constexpr int WCH = 128;          // K columns staged per chunk (4 k-steps)
constexpr int WKS = WCH / 32;     // k-steps per chunk
constexpr int WT = 2;             // 16-column tiles per wave: each operand read from LDS feeds WT multiplies
constexpr int WRC = 1;            // chunks of fragments in flight per wave
constexpr int WSPF = WRC * WKS * WT;   // fragment loads in flight per wave
constexpr int WMAXR = 128;        // max activation rows of one expert in a wide group
constexpr int WLDA = WCH + 8;     // LDS row stride (halves): rows of a chunk start on different banks

struct WEx {
  const h16x8* w;      // packed weights: fragment (tile t, k-step s) at ((t * K/32) + s) * 64
  const h16* a;        // activation rows [S][lda]; the unit's K range [kc K/ks, (kc+1) K/ks) is read
  int lda;
  const h16* bias;     // E_BIAS16 / E_GELU16 bias [N]
  void* out;           // E_PART: float [ks][S][N]; E_PART16: h16 (as SEx); otherwise h16 (below)
  int S;               // activation rows (1 .. WMAXR)
  int pack, hrows;     // E_PART16: as SEx
  int nsplit;          // E_BIAS16: column n goes to block n / nsplit, stored [blocks][S][nsplit] (0: [S][N])
  const int* ids;      // row i of the operand is a[max(ids[i * ids_stride], 0)] (a gather), or row i (null)
  int ids_stride;
};

struct WArgs {
  WEx ex[4];
  int nex, N, K, ks, wg_per_kc;
  int gelu_r16;        // E_GELU16: as SArgs
  int pair;            // entries e and e + nex/2 stream the same weights (two request groups of one
                       // expert): their workgroups for a unit run side by side on one XCD
  int map;             // workgroup order (set by launch_wide): MAP_PLAIN, MAP_PAIR or MAP_XCD
};

// Workgroup -> (entry, k-split, tile group) orders.  Workgroups go to the 8 XCDs round robin,
// each XCD with its own L2, starting from an XCD that depends on the dispatches before the launch:
// workgroups b and b' share an XCD when b = b' mod 8 (below, "XCD x" is the XCD of the workgroups
// b = x mod 8, whichever it is).
//   MAP_PLAIN: entry-major.
//   MAP_PAIR:  workgroups b and b + 8 take the same unit of entries e and e + nex/2.
//   MAP_XCD:   (split-K) XCD x takes every unit of the (entry, k-split) combinations x, x + 8, ...:
//              each XCD reads the operand rows of its own K ranges only, instead of every XCD
//              reading all of them (W2's 128 rows x 24576 columns are 6.3 MB an entry), and with
//              nex/2 * ks a multiple of 8 the two groups' combinations of one weight range share
//              an XCD.
enum { MAP_PLAIN = 0, MAP_PAIR = 1, MAP_XCD = 2 };

template <int EPI, int NG, int WV>
__global__ void __launch_bounds__(WV * 64) k_wide(WArgs a) {
  extern __shared__ __align__(16) h16 lds[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int b = blockIdx.x;
  const int per_ex = a.ks * a.wg_per_kc;
  int e, kc, tg;
  if (a.map == MAP_XCD) {
    const int x = b & 7, j = b >> 3;
    const int cl = j / a.wg_per_kc;
    const int combo = x + 8 * cl;
    tg = j - cl * a.wg_per_kc;
    e = combo / a.ks;
    kc = combo - e * a.ks;
  } else {
    if (a.map == MAP_PAIR) {
      // workgroups b and b + 8 (dispatched together, on the same XCD) take the same unit of the
      // two groups, so the second reads the weight fragments the first has just brought into the
      // XCD's L2 instead of from HBM
      const int lo = b & 7, hi = b >> 3;
      b = (((hi >> 1) << 3) | lo) + (hi & 1) * (a.nex / 2) * per_ex;
    }
    e = b / per_ex;
    b -= e * per_ex;
    kc = b / a.wg_per_kc;
    tg = b - kc * a.wg_per_kc;
  }
  const WEx& ex = a.ex[e];
  const int S = ex.S;
  const int ksteps = a.K / 32;
  const int KCW = a.K / a.ks, nsteps = KCW / 32, nchunk = KCW / WCH;
  const int t0 = (tg * WV + wave) * WT;               // this wave's WT adjacent 16-column tiles
  const int k0 = kc * KCW;
  // staging of one chunk: vector idx = u * nt + thread, row idx / 16, columns (idx % 16) * 8 .. +7;
  // indices past the rows re-read the last vector (every load unconditional, see Stage)
  constexpr int NT = WV * 64;
  constexpr int NVR = WCH / 8;                        // 16-byte vectors per row of a chunk
  constexpr int NSV = (NG * 16 * NVR + NT - 1) / NT;  // vectors per thread at the most rows
  const int total = S * NVR;
  // each staging slot's element offset in the operand, the same at every chunk (a gathered row's
  // index is read once)
  size_t soff[NSV];
#pragma unroll
  for (int u = 0; u < NSV; ++u) {
    const int idx = min(u * NT + (int)threadIdx.x, total - 1);
    const int i = idx / NVR, kk = (idx - i * NVR) * 8;
    const size_t src = ex.ids ? (size_t)max(ex.ids[(size_t)i * ex.ids_stride], 0) : (size_t)i;
    soff[u] = src * ex.lda + kk;
  }
  h16x8 st[NSV];
  auto load_chunk = [&](int c) {
    const h16* base = ex.a + k0 + c * WCH;
#pragma unroll
    for (int u = 0; u < NSV; ++u) st[u] = *(const h16x8*)(base + soff[u]);
  };
  auto place_chunk = [&](h16* buf) {
#pragma unroll
    for (int u = 0; u < NSV; ++u) {
      const int idx = min(u * NT + (int)threadIdx.x, total - 1);
      const int i = idx / NVR, kk = (idx - i * NVR) * 8;
      *(h16x8*)(buf + i * WLDA + kk) = st[u];
    }
  };
  // the wave's fragments, k-step by k-step, the WT tiles of a k-step together; past the last
  // k-step the pointers stay there, so the ring's surplus refills re-read lines just fetched
  const h16x8* lw = ex.w + ((size_t)t0 * ksteps + (size_t)kc * nsteps) * 64 + lane;
  const size_t tstride = (size_t)ksteps * 64;         // next tile, same k-step
  int lleft = nsteps * WT;
  auto issue = [&](int u) -> h16x8 {
    const h16x8 v = __builtin_nontemporal_load(lw + u * tstride);
    if (u == WT - 1) {
      const bool adv = lleft > WT;
      lw += adv ? 64 : 0;
      lleft -= adv ? WT : 0;
    }
    return v;
  };
  const int col = lane & 15, rbase = 4 * (lane >> 4);
  float bias[WT] = {};
  if constexpr (EPI == E_BIAS16 || EPI == E_GELU16) {
#pragma unroll
    for (int u = 0; u < WT; ++u) bias[u] = (float)ex.bias[(t0 + u) * 16 + col];
  }
  // operand chunk 0 first, then the weight prefetch (independent of it), then LDS
  load_chunk(0);
  __builtin_amdgcn_sched_barrier(0);
  h16x8 ring[WSPF];
#pragma unroll
  for (int p = 0; p < WSPF; ++p) {
    ring[p] = issue(p % WT);
    // issued in slot order: each multiply then waits for its own slot alone (with the order left
    // free, slot 0 went out seventh and the first multiply waited for the whole ring)
    __builtin_amdgcn_sched_barrier(0);
  }
  h16* buf0 = lds;
  h16* buf1 = lds + (size_t)S * WLDA;
  place_chunk(buf0);
  lds_barrier();
  const int row = lane & 15, kg = lane >> 4;
  f32x4 acc[WT][NG];
#pragma unroll
  for (int u = 0; u < WT; ++u)
#pragma unroll
    for (int g = 0; g < NG; ++g) acc[u][g] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // lanes of rows past S read row 0: their products land in output rows that are never stored
  // (every row group is multiplied, which keeps the loop free of branches)
  int roff[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) roff[g] = (g * 16 + row < S ? g * 16 + row : 0) * WLDA + kg * 8;
  const h16x8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  // WRC chunks per ring cycle: slot p holds tile p % WT of k-step (p / WT) % WKS of chunk
  // c0 + p / (WT WKS)
  for (int c0 = 0; c0 < nchunk; c0 += WRC) {
#pragma unroll
    for (int h = 0; h < WRC; ++h) {
      const int c = c0 + h;
      // past the last chunk (a count that is not a multiple of WRC) zero fragments multiply the last
      // chunk's rows, which are finite (0 x NaN from a buffer never written would poison the sums);
      // the loop keeps no branches
      const h16* cur = (min(c, nchunk - 1) & 1) ? buf1 : buf0;
      h16* nxt = (c & 1) ? buf0 : buf1;
      load_chunk(min(c + 1, nchunk - 1));
#pragma unroll
      for (int q = 0; q < WKS; ++q) {
        const int p0 = (h * WKS + q) * WT;
        h16x8 bf[WT];
#pragma unroll
        for (int u = 0; u < WT; ++u) bf[u] = (WRC == 1 || c < nchunk) ? ring[p0 + u] : zero8;
        // one k-step at a time: each row group's operand read once, multiplied by the WT fragments
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          const h16x8 av = *(const h16x8*)(cur + roff[g] + q * 32);
#pragma unroll
          for (int u = 0; u < WT; ++u) acc[u][g] = mfma_f16(av, bf[u], acc[u][g]);
        }
#pragma unroll
        for (int u = 0; u < WT; ++u) ring[p0 + u] = issue(u);
        // left free, the scheduler hoists every read of the chunk ahead of the multiplies and runs
        // out of registers
        __builtin_amdgcn_sched_barrier(0);
      }
      // chunk c + 1 goes to the other buffer (nobody reads it: every wave finished chunk c - 1
      // before the last barrier); one barrier orders the stores before chunk c + 1's reads
      if (c + 1 < nchunk) place_chunk(nxt);
      lds_barrier();
    }
  }
  // epilogue: rows g * 16 + rbase + q of column (t0 + u) * 16 + col
#pragma unroll
  for (int u = 0; u < WT; ++u) {
    const int n = (t0 + u) * 16 + col;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (g * 16 >= S) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = g * 16 + rbase + q;
        if (r >= S) continue;
        const float v = acc[u][g][q];
        if constexpr (EPI == E_PART) {
          ((float*)ex.out)[((size_t)kc * S + r) * a.N + n] = v;
        } else if constexpr (EPI == E_PART16) {
          const int hr = ex.hrows > 0 ? ex.hrows : S, hb = r / hr, rr = r - hb * hr;
          h16* o = (h16*)ex.out + ((size_t)kc * (S / hr) + hb) * hr * a.N;
          o[ex.pack ? frag_index(rr, n, hr) : (size_t)rr * a.N + n] = (h16)v;
        } else if constexpr (EPI == E_BIAS16) {
          if (ex.nsplit > 0) {
            const int part = n / ex.nsplit, nn = n - part * ex.nsplit;
            ((h16*)ex.out)[((size_t)part * S + r) * ex.nsplit + nn] = (h16)(v + bias[u]);
          } else {
            ((h16*)ex.out)[(size_t)r * a.N + n] = (h16)(v + bias[u]);
          }
        } else {
          const float w = v + bias[u];
          ((h16*)ex.out)[(size_t)r * a.N + n] = (h16)gelu_erf(a.gelu_r16 ? r16(w) : w);
        }
      }
    }
  }
}

size_t wide_lds(int S_max) { return (size_t)2 * S_max * WLDA * 2; }

template <int EPI, int NG, int WV>
int launch_wide_k(const WArgs& a, size_t lds, hipStream_t st) {
  static unsigned long long attr_set = 0;
  int dev = 0;
  CFH_HIP(hipGetDevice(&dev));
  if (dev < 64 && !(attr_set & (1ull << dev))) {
    CFH_HIP(hipFuncSetAttribute((const void*)k_wide<EPI, NG, WV>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                150 * 1024));
    attr_set |= 1ull << dev;
  }
  const long long wgs = (long long)a.nex * a.ks * a.wg_per_kc;
  hipLaunchKernelGGL((k_wide<EPI, NG, WV>), dim3((unsigned)wgs), dim3(WV * 64), lds, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// Shape checks of a wide launch (also used by the plan): CFH_OK when every unit of wv waves covers
// whole tiles, every k-split a whole number of chunks, and the rows fit.
int wide_check(const WArgs& a, int wv, int S_max) {
  if (a.nex < 1 || a.nex > 4 || a.N <= 0 || a.N % 16 || a.ks <= 0 || a.K % a.ks || (a.K / a.ks) % WCH)
    return CFH_E_UNSUPPORTED;
  if ((wv != 4 && wv != 6 && wv != 8 && wv != 12) || (a.N / 16) % (WT * wv) || S_max < 1 || S_max > WMAXR ||
      wide_lds(S_max) > 150 * 1024)
    return CFH_E_UNSUPPORTED;
  if (a.pair && a.nex % 2) return CFH_E_UNSUPPORTED;
  return CFH_OK;
}

// Waves per workgroup of a wide launch over `units` units of `tiles` column tiles: the count
// (WT tiles a wave, dividing tiles) that loads the busiest CU least -- rounds of 256 workgroups
// times waves a workgroup -- preferring fewer waves a workgroup on ties.
int wide_wv(int tiles, int units) {
  constexpr int CUS = 256;
  int best = 0;
  long long best_load = 0;
  for (int wv : {4, 6, 8, 12}) {
    if (tiles % (WT * wv)) continue;
    const long long wgs = (long long)units * tiles / (WT * wv);
    const long long load = (wgs + CUS - 1) / CUS * wv;
    if (!best || load < best_load) {
      best = wv;
      best_load = load;
    }
  }
  return best;
}


template <int EPI>
int launch_wide(const WArgs& a0, int wv, hipStream_t st) {
  WArgs a = a0;
  int S_max = 0;
  for (int e = 0; e < a.nex; ++e) S_max = std::max(S_max, a.ex[e].S);
  if (wide_check(a, wv, S_max)) return CFH_E_UNSUPPORTED;
  for (int e = 0; e < a.nex; ++e)
    if (a.ex[e].S < 1 || a.ex[e].lda < a.K || !a.ex[e].w || !a.ex[e].a || !a.ex[e].out) return CFH_E_INVALID;
  a.wg_per_kc = (a.N / 16) / (WT * wv);
  // the side-by-side order needs a whole number of 8-workgroup runs per half (narrow widths such as
  // d = 640 have 5 a k-split: their paired launches keep the plain order, still one launch for both)
  const bool pair_runs = a.pair && ((long long)(a.nex / 2) * a.ks * a.wg_per_kc) % 8 == 0;
  if (a.ks > 1 && (a.nex * a.ks) % 8 == 0 && (!a.pair || ((a.nex / 2) * a.ks) % 8 == 0))
    a.map = MAP_XCD;
  else
    a.map = pair_runs ? MAP_PAIR : MAP_PLAIN;
  const size_t lds = wide_lds(S_max);
  const int ng = (S_max + 15) / 16;
#define CFH_WIDE(G)                                                                 \
  if (ng <= G) {                                                                    \
    switch (wv) {                                                                   \
      case 4: return launch_wide_k<EPI, G, 4>(a, lds, st);                          \
      case 6: return launch_wide_k<EPI, G, 6>(a, lds, st);                          \
      case 8: return launch_wide_k<EPI, G, 8>(a, lds, st);                          \
      default: return launch_wide_k<EPI, G, 12>(a, lds, st);                        \
    }                                                                               \
  }
  CFH_WIDE(2) CFH_WIDE(4) CFH_WIDE(8)
#undef CFH_WIDE
  return CFH_E_UNSUPPORTED;
}

// Self attention of a wide group (causal, or with no mask), one workgroup per (entry, request,
// head): the request's Sr rows of q, k, v (columns of head h of the [S][3d] rows) staged in LDS,
// then `attend` (the narrow kernel's attention, same arithmetic), written as fp16 rows [S][d] of
// the attention output.
struct SelfArgs {
  const h16* qkv[4];   // [S][3d]
  h16* out[4];         // [S][d]
  int S[4], Sr[4];     // rows, rows per request
  int nex, R, H, d, hd;
  int bidir;           // 0: causal (the flow's draft rows); 1: no mask (the VAE's sequences)
};

constexpr int SAT = 256;          // threads of a self-attention workgroup

__global__ void __launch_bounds__(SAT) k_self_attn(SelfArgs a) {
  extern __shared__ __align__(16) h16 sm[];
  int b = blockIdx.x;
  const int h = b % a.H;
  b /= a.H;
  const int j = b % a.R, e = b / a.R;
  const int Sr = a.Sr[e], hd = a.hd, d = a.d;
  if ((j + 1) * Sr > a.S[e]) return;                  // (a request the group does not hold)
  const h16* src = a.qkv[e] + (size_t)j * Sr * 3 * d + h * hd;
  h16* sq = sm;
  h16* sk = sq + Sr * hd;
  h16* sv = sk + Sr * hd;
  float* P = (float*)(sv + Sr * hd);                  // [Sr][Sr]
  const int nv = hd / 8;
  for (int idx = threadIdx.x; idx < 3 * Sr * nv; idx += blockDim.x) {
    const int part = idx / (Sr * nv), rem = idx - part * Sr * nv;
    const int i = rem / nv, c = (rem - i * nv) * 8;
    *(h16x8*)(sq + (size_t)(part * Sr + i) * hd + c) = *(const h16x8*)(src + (size_t)i * 3 * d + part * d + c);
  }
  lds_barrier();
  attend(Sr, Sr, Sr, Sr, hd, hd, !a.bidir, sq, sk, sv, P, a.out[e] + (size_t)j * Sr * d + h * hd, d);
}

int launch_self_attn(const SelfArgs& a, hipStream_t st) {
  if (a.hd % 8 || a.hd <= 0 || a.nex < 1 || a.nex > 4) return CFH_E_UNSUPPORTED;
  int Srm = 0;
  for (int e = 0; e < a.nex; ++e) {
    if (a.Sr[e] < 1 || a.Sr[e] > 16 || a.S[e] > a.R * a.Sr[e]) return CFH_E_UNSUPPORTED;
    Srm = std::max(Srm, a.Sr[e]);
  }
  const size_t lds = (size_t)3 * Srm * a.hd * 2 + (size_t)Srm * Srm * 4;
  if (lds > 64 * 1024) return CFH_E_UNSUPPORTED;
  hipLaunchKernelGGL(k_self_attn, dim3((unsigned)(a.nex * a.R * a.H)), dim3(SAT), lds, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// Cross attention of a wide group whose heads do not fold (head widths such as 80: two heads an
// MFMA k-chunk), one workgroup per (expert, request, head): the request's Sr rows of q (columns of
// head h of the [S][d] rows, bias included), its C context rows of K and V (block l's [2][Ct][d]
// image, the request's rows [j C, j C + C)), staged in LDS, then `attend` without a mask, written
// as fp16 rows [S][d] of the attention output.
struct CrossArgs {
  const h16* q[4];     // [S][d]
  const h16* kv[4];    // [2][Ct][d]: K rows then V rows
  h16* out[4];         // [S][d]
  int S[4], Sr[4], Ct[4];
  int nex, R, H, d, hd, C;
};

__global__ void __launch_bounds__(SAT) k_cross_attn(CrossArgs a) {
  extern __shared__ __align__(16) h16 sm[];
  int b = blockIdx.x;
  const int h = b % a.H;
  b /= a.H;
  const int j = b % a.R, e = b / a.R;
  const int Sr = a.Sr[e], C = a.C, hd = a.hd, d = a.d;
  if ((j + 1) * Sr > a.S[e] || (j + 1) * C > a.Ct[e]) return;   // (a request the group does not hold)
  const h16* qs = a.q[e] + (size_t)j * Sr * d + h * hd;
  const h16* ks = a.kv[e] + (size_t)j * C * d + h * hd;
  const h16* vs = ks + (size_t)a.Ct[e] * d;
  h16* sq = sm;
  h16* sk = sq + Sr * hd;
  h16* sv = sk + C * hd;
  float* P = (float*)(sv + C * hd);                   // [Sr][C]
  const int nv = hd / 8;
  for (int idx = threadIdx.x; idx < (Sr + 2 * C) * nv; idx += blockDim.x) {
    const int i = idx / nv, c = (idx - i * nv) * 8;
    const h16* src = i < Sr ? qs + (size_t)i * d : i < Sr + C ? ks + (size_t)(i - Sr) * d : vs + (size_t)(i - Sr - C) * d;
    *(h16x8*)(sq + (size_t)i * hd + c) = *(const h16x8*)(src + c);
  }
  lds_barrier();
  attend(Sr, C, Sr, C, hd, hd, false, sq, sk, sv, P, a.out[e] + (size_t)j * Sr * d + h * hd, d);
}

size_t cross_attn_lds(int Sr, int C, int hd) { return (size_t)(Sr + 2 * C) * hd * 2 + (size_t)Sr * C * 4; }

int launch_cross_attn(const CrossArgs& a, hipStream_t st) {
  if (a.hd % 8 || a.hd <= 0 || a.nex < 1 || a.nex > 4 || a.C < 1 || a.C > 16) return CFH_E_UNSUPPORTED;
  int Srm = 0;
  for (int e = 0; e < a.nex; ++e) {
    if (a.Sr[e] < 1 || a.Sr[e] > 16 || a.S[e] > a.R * a.Sr[e] || a.Ct[e] > a.R * a.C) return CFH_E_UNSUPPORTED;
    Srm = std::max(Srm, a.Sr[e]);
  }
  const size_t lds = cross_attn_lds(Srm, a.C, a.hd);
  if (lds > 64 * 1024) return CFH_E_UNSUPPORTED;
  hipLaunchKernelGGL(k_cross_attn, dim3((unsigned)(a.nex * a.R * a.H)), dim3(SAT), lds, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// The context rows' LayerNorm of every block, once per draft: rows[e][l][c] =
// fp16((ctx[c] - mean_c) rstd_c g_l + b_l) with the row moments the ROWS kernel left in mom (the
// narrow cross K/V stream applies the same formula while staging).
struct CtxLnArgs {
  const h16* ctx;      // [Ct][d]
  const float* mom;    // [Ct][2]
  const h16* g0[4];    // block 0's context_norm weight of each expert; block l at + l * vstride bytes
  const h16* b0[4];
  h16* out[4];         // [L][Ct][d]
  long long vstride;
  int nex, nl, Ct, d;
};

__global__ void __launch_bounds__(256) k_ctx_ln(CtxLnArgs a) {
  const int nv = a.d / 8;
  const size_t per_l = (size_t)a.Ct * nv, per_e = per_l * a.nl, total = per_e * a.nex;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int e = (int)(i / per_e);
    size_t r = i - (size_t)e * per_e;
    const int l = (int)(r / per_l);
    r -= (size_t)l * per_l;
    const int c = (int)(r / nv), k = (int)(r - (size_t)c * nv) * 8;
    const h16* gw = (const h16*)((const char*)a.g0[e] + (size_t)l * a.vstride);
    const h16* gb = (const h16*)((const char*)a.b0[e] + (size_t)l * a.vstride);
    const h16x8 xv = *(const h16x8*)(a.ctx + (size_t)c * a.d + k);
    const h16x8 gv = *(const h16x8*)(gw + k);
    const h16x8 bv = *(const h16x8*)(gb + k);
    const float mu = a.mom[2 * c], rs = a.mom[2 * c + 1];
    h16x8 o;
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] = (h16)(((float)xv[t] - mu) * rs * (float)gv[t] + (float)bv[t]);
    *(h16x8*)(a.out[e] + ((size_t)l * a.Ct + c) * a.d + k) = o;
  }
}

}  // namespace
