// Pass A of the two-pass candidate head on MI355X (FlowDrafterProposer._candidates,
// cf/vllm_plugin/flow_proposer.py:1142-1165).  The scores come from the ordinary head kernel
// (fp16 logits of every depth's marginal hidden over the whole shortlist, and each row's
// log-sum-exp); this file picks each request's M candidate columns:
//   value[j] = max over the request's n rows d of (logits[d][j] - lse[d])   (fp32)
// (shared: the best per-depth log-prob; n = 1 gives the per-depth set, the order of the raw logits),
// the M largest values with ties to the lower column, written in ascending column order.
// The values become order-preserving 32-bit keys in `ws` (a wide grid; rows padded to 4 keys);
// then one 1024-thread workgroup per request finds the bits every key shares, runs a
// most-significant-digit-first radix select over the rest (12-bit digits, histograms in LDS) that
// finds the M-th largest key and how many ties at it belong to the M, and compacts in column order
// by 256-column segments (ballot counts, workgroup scans of the segment counts, ballot ranks).
// No sort and no atomics on global memory; deterministic.
#include <math.h>

#include "cfh_kernels.h"

namespace {

constexpr int CT = 1024;   // threads per request

__device__ __forceinline__ unsigned order_key(float v) {
  const unsigned u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive scan of one int per thread over the workgroup; *total = the sum.  Each wave scans its
// lanes with shuffles, the 16 wave totals go through LDS: two barriers, not two per doubling step.
__device__ int block_exscan(int v, int* buf, int* total) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(incl, off);
    if (lane >= off) incl += u;
  }
  if (lane == 63) buf[wave] = incl;
  __syncthreads();
  int base = 0, sum = 0;
  for (int w = 0; w < CT / 64; ++w) {
    const int x = buf[w];
    base += w < wave ? x : 0;
    sum += x;
  }
  *total = sum;
  __syncthreads();   // buf is reused by the next scan
  return base + incl - v;
}

struct CandArgs {
  const unsigned short* logits;   // fp16 [B * n][ld]
  const float* lse;               // [B * n]
  const int* sl;                  // [Vs] or null
  int* cand_local;                // [B][M]
  int* cand_global;               // [B][M] or null
  unsigned* keys;                 // ws [B][Vp], Vp = Vs rounded up to 4 (16-byte rows)
  long long ld;
  int n, Vs, M, B;
};

__host__ __device__ constexpr int padded_vs(int Vs) { return (Vs + 3) & ~3; }
// column blocks of k_cand_keys (1024 columns each); after the keys, ws holds each block's AND and
// OR of its keys: masks [B][key_blocks][2]
__host__ __device__ constexpr int key_blocks(int Vs) { return (Vs + 1023) / 1024; }

// keys[b][j] for 4 columns a thread, grid (B, column blocks): coalesced and spread over the chip;
// each block also writes the AND and the OR of its keys (order-free, so still deterministic)
__global__ void __launch_bounds__(256) k_cand_keys(CandArgs a) {
  __shared__ unsigned red[2][4];
  const int b = blockIdx.x;
  unsigned kand = ~0u, kor = 0u;
  for (int q = 0; q < 4; ++q) {
    const int j = (blockIdx.y * 4 + q) * 256 + threadIdx.x;
    if (j >= a.Vs) break;
    float v = -INFINITY;
    for (int d = 0; d < a.n; ++d) {
      const size_t r = (size_t)b * a.n + d;
      v = fmaxf(v, (float)__builtin_bit_cast(_Float16, a.logits[r * a.ld + j]) - a.lse[r]);
    }
    const unsigned k = order_key(v);
    a.keys[(size_t)b * padded_vs(a.Vs) + j] = k;
    kand &= k;
    kor |= k;
  }
  for (int off = 32; off > 0; off >>= 1) {
    kand &= (unsigned)__shfl_xor((int)kand, off);
    kor |= (unsigned)__shfl_xor((int)kor, off);
  }
  if ((threadIdx.x & 63) == 0) {
    red[0][threadIdx.x >> 6] = kand;
    red[1][threadIdx.x >> 6] = kor;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned* m = a.keys + (size_t)a.B * padded_vs(a.Vs) + ((size_t)b * key_blocks(a.Vs) + blockIdx.y) * 2;
    m[0] = red[0][0] & red[0][1] & red[0][2] & red[0][3];
    m[1] = red[1][0] | red[1][1] | red[1][2] | red[1][3];
  }
}

// Radix select over the bits below the keys' common prefix, 12 bits a pass (4096 bins; the last
// pass takes what is left): the bits every key shares (the sign and most of the exponent of the
// log-probabilities) would put all keys in a few bins and serialise the histogram atomics on
// them.  Each pass counts only the keys that match the digits chosen so far; the digit holding the
// M-th largest key is found by a workgroup scan over the bins (thread t owns bins 4t .. 4t+3 from
// the top).  `each` visits the thread's keys.
template <typename Each>
__device__ void select_digit(Each& each, unsigned prefix, unsigned pmask, int shift, int bins, int* hist, int* scan,
                             unsigned* s_prefix, int* s_rem) {
  const int t = threadIdx.x;
  for (int i = t; i < bins; i += CT) hist[i] = 0;
  __syncthreads();
  const unsigned dmask = (unsigned)bins - 1;
  each([&](unsigned k) {
    if ((k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & dmask], 1);
  });
  __syncthreads();
  const int per = bins / CT > 0 ? bins / CT : 1;            // 4 bins a thread at 4096, else 1
  int cnt[4] = {0, 0, 0, 0}, sum = 0;
  for (int i = 0; i < per; ++i) {
    const int bin = bins - 1 - (t * per + i);
    cnt[i] = bin >= 0 ? hist[bin] : 0;
    sum += cnt[i];
  }
  int tot;
  int above = block_exscan(sum, scan, &tot);
  const int rem = *s_rem;
  __syncthreads();
  for (int i = 0; i < per; ++i) {
    const int bin = bins - 1 - (t * per + i);
    if (bin >= 0 && above < rem && above + cnt[i] >= rem) {
      *s_prefix = prefix | ((unsigned)bin << shift);
      *s_rem = rem - above;
    }
    above += cnt[i];
  }
  __syncthreads();
}

// Every pass reads the keys as 16-byte vectors (4 columns a lane; consecutive lanes, consecutive
// vectors) in batches of KB loads a thread issues together: one workgroup per request is bound by
// the loads it keeps in flight.  The compaction works on 256-column segments, one wave each: ballot
// counts per segment, then segment offsets by two workgroup scans, then each column's output slot
// from the ballots of the lanes below it.  A wave loads all its segments' keys in one batch (up to
// 65,536 columns), and the shortlist ids are gathered in a last pass over the M outputs: a load
// issued after stores waits for them (the wave's memory counter is in order).
constexpr int KB = 8;         // vectors in flight per thread per batch
constexpr int SEGB = 16;      // segments in flight per wave
constexpr int MAXSEG = 1024;  // 256-column segments: Vs <= 262,144

__global__ void __launch_bounds__(CT) k_cand_select(CandArgs a) {
  __shared__ int hist[4096];
  __shared__ int scan[CT];
  __shared__ int sg_a[MAXSEG], sg_b[MAXSEG];
  __shared__ unsigned s_prefix;
  __shared__ int s_rem;
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int nv = padded_vs(a.Vs) / 4;
  const uint4* keys = (const uint4*)(a.keys + (size_t)b * padded_vs(a.Vs));
  auto each = [&](auto&& f) {
    for (int v0 = t; v0 < nv; v0 += CT * KB) {
      uint4 kb[KB];
#pragma unroll
      for (int u = 0; u < KB; ++u) kb[u] = keys[min(v0 + u * CT, nv - 1)];   // (past nv: never used)
#pragma unroll
      for (int u = 0; u < KB; ++u) {
        const int j = 4 * (v0 + u * CT);
        if (j < a.Vs) f(kb[u].x);
        if (j + 1 < a.Vs) f(kb[u].y);
        if (j + 2 < a.Vs) f(kb[u].z);
        if (j + 3 < a.Vs) f(kb[u].w);
      }
    }
  };
  // the keys' common prefix: bits where the AND and the OR of every key agree (from the key
  // blocks' masks)
  unsigned kand = ~0u, kor = 0u;
  const unsigned* masks = a.keys + (size_t)a.B * padded_vs(a.Vs) + (size_t)b * key_blocks(a.Vs) * 2;
  for (int i = t; i < key_blocks(a.Vs); i += CT) {
    kand &= masks[2 * i];
    kor |= masks[2 * i + 1];
  }
  for (int off = 32; off > 0; off >>= 1) {
    kand &= (unsigned)__shfl_xor((int)kand, off);
    kor |= (unsigned)__shfl_xor((int)kor, off);
  }
  if (lane == 0) {
    scan[wave] = (int)kand;
    scan[CT / 64 + wave] = (int)kor;
  }
  __syncthreads();
  kand = ~0u;
  kor = 0u;
  for (int w = 0; w < CT / 64; ++w) {
    kand &= (unsigned)scan[w];
    kor |= (unsigned)scan[CT / 64 + w];
  }
  __syncthreads();
  const unsigned diff = kand ^ kor;
  // bits [lo, 32) are fixed; lo = 0 when every key is equal (then all M come from the ties)
  int lo = diff ? 32 - __clz(diff) : 0;
  unsigned pmask = lo >= 32 ? 0u : ~((1u << lo) - 1u);
  if (t == 0) { s_prefix = kand & pmask; s_rem = a.M; }
  __syncthreads();
  while (lo > 0) {
    const int w = min(12, lo), shift = lo - w;
    select_digit(each, s_prefix, pmask, shift, 1 << w, hist, scan, &s_prefix, &s_rem);
    pmask |= ((1u << w) - 1u) << shift;
    lo = shift;
  }
  const unsigned T = s_prefix;
  const int need = s_rem;   // ties at T that belong to the M (lowest columns first)
  // compaction in column order by 256-column segments (lane l holds columns 4l .. 4l+3)
  const int nseg = (nv + 63) / 64;
  const unsigned long long below = (1ull << lane) - 1ull;
  auto segments = [&](auto&& f) {   // f(segment, first column, keys) on every lane of the wave
    for (int s0 = wave; s0 < nseg; s0 += (CT / 64) * SEGB) {
      uint4 kk[SEGB];
#pragma unroll
      for (int u = 0; u < SEGB; ++u) kk[u] = keys[min((s0 + u * (CT / 64)) * 64 + lane, nv - 1)];
#pragma unroll
      for (int u = 0; u < SEGB; ++u) {
        const int sg = s0 + u * (CT / 64);
        if (sg < nseg) f(sg, (sg * 64 + lane) * 4, kk[u]);   // (wave-uniform)
      }
    }
  };
  segments([&](int sg, int j, uint4 k4) {
    const unsigned k[4] = {k4.x, k4.y, k4.z, k4.w};
    int gt = 0, eq = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bool ok = j + q < a.Vs;
      gt += __popcll(__ballot(ok && k[q] > T));
      eq += __popcll(__ballot(ok && k[q] == T));
    }
    if (lane == 0) { sg_a[sg] = gt; sg_b[sg] = eq; }
  });
  __syncthreads();
  // segment offsets: thread t owns segments [g0, g1); sg_b becomes the ties before the segment,
  // sg_a the output slot of its first column
  const int sp = (nseg + CT - 1) / CT;
  const int g0 = min(t * sp, nseg), g1 = min(g0 + sp, nseg);
  int eq_own = 0;
  for (int g = g0; g < g1; ++g) eq_own += sg_b[g];
  int tot;
  int eq_run = block_exscan(eq_own, scan, &tot);
  int out_own = 0;
  for (int g = g0; g < g1; ++g) out_own += sg_a[g] + min(max(need - eq_run, 0), sg_b[g]), eq_run += sg_b[g];
  int out_run = block_exscan(out_own, scan, &tot);
  eq_run -= eq_own;
  for (int g = g0; g < g1; ++g) {
    const int gt = sg_a[g], eq = sg_b[g];
    sg_a[g] = out_run;
    sg_b[g] = eq_run;
    out_run += gt + min(max(need - eq_run, 0), eq);
    eq_run += eq;
  }
  __syncthreads();
  int* cl = a.cand_local + (size_t)b * a.M;
  int* cg = a.cand_global ? a.cand_global + (size_t)b * a.M : nullptr;
  segments([&](int sg, int j, uint4 k4) {
    const unsigned k[4] = {k4.x, k4.y, k4.z, k4.w};
    bool eqb[4], take[4];
    int eq_rank = sg_b[sg];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      eqb[q] = j + q < a.Vs && k[q] == T;
      eq_rank += __popcll(__ballot(eqb[q]) & below);
    }
    int pos = sg_a[sg];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      take[q] = (j + q < a.Vs && k[q] > T) || (eqb[q] && eq_rank < need);
      eq_rank += eqb[q];
      pos += __popcll(__ballot(take[q]) & below);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (take[q]) cl[pos++] = j + q;
    }
  });
  if (cg) {   // global ids of the candidates (the barrier makes the workgroup's stores visible)
    __syncthreads();
    for (int i = t; i < a.M; i += CT) {
      const int c = cl[i];
      cg[i] = a.sl ? a.sl[c] : c;
    }
  }
}

}  // namespace

extern "C" {

int64_t cfh_cand_ws_bytes(int B, int Vs) {
  if (B < 0 || Vs < 0) return -1;
  return (int64_t)B * padded_vs(Vs) * 4 + (int64_t)B * key_blocks(Vs) * 8;
}

int cfh_cand_topm(const void* logits, long long ld, const float* lse, int B, int n, int Vs, int M, const int32_t* sl,
                  int32_t* cand_local, int32_t* cand_global, void* ws, void* stream) {
  if (B == 0) return CFH_OK;
  if (!logits || !lse || !cand_local || !ws || B < 0 || n < 1 || Vs < 1 || M < 1 || M > Vs || ld < Vs)
    return CFH_E_INVALID;
  if ((uintptr_t)ws & 15) return CFH_E_INVALID;
  if (Vs > 256 * MAXSEG) return CFH_E_UNSUPPORTED;
  CandArgs a = {(const unsigned short*)logits, lse, sl, cand_local, cand_global, (unsigned*)ws, ld, n, Vs, M, B};
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_cand_keys, dim3(B, key_blocks(Vs)), dim3(256), 0, st, a);
  CFH_LAUNCH_CHECK();
  hipLaunchKernelGGL(k_cand_select, dim3(B), dim3(CT), 0, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

}  // extern "C"
