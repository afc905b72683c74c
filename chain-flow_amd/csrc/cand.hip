// Pass A of the two-pass candidate head on MI355X (FlowDrafterProposer._candidates,
// cf/vllm_plugin/flow_proposer.py:1142-1165).  The scores come from the ordinary head kernel
// (fp16 logits of every depth's marginal hidden over the whole shortlist, and each row's
// log-sum-exp); this file picks each request's M candidate columns:
//   value[j] = max over the request's n rows d of (logits[d][j] - lse[d])   (fp32)
// (shared: the best per-depth log-prob; n = 1 gives the per-depth set, the order of the raw logits),
// the M largest values with ties to the lower column, written in ascending column order.
// The values become order-preserving 32-bit keys in `ws` (a wide grid); then one 1024-thread
// workgroup per request runs a most-significant-digit-first radix select (histograms in LDS) that
// finds the M-th largest key and how many ties at it belong to the M, and a workgroup scan in
// column order compacts.  No sort and no atomics on global memory; deterministic.
#include <math.h>

#include "cfh_kernels.h"

namespace {

constexpr int CT = 1024;   // threads per request

__device__ __forceinline__ unsigned order_key(float v) {
  const unsigned u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive scan of one int per thread over the workgroup (LDS, Hillis-Steele); *total = the sum.
__device__ int block_exscan(int v, int* buf, int* total) {
  const int t = threadIdx.x;
  buf[t] = v;
  __syncthreads();
  for (int off = 1; off < CT; off <<= 1) {
    const int add = t >= off ? buf[t - off] : 0;
    __syncthreads();
    buf[t] += add;
    __syncthreads();
  }
  const int incl = buf[t];
  *total = buf[CT - 1];
  __syncthreads();
  return incl - v;
}

struct CandArgs {
  const unsigned short* logits;   // fp16 [B * n][ld]
  const float* lse;               // [B * n]
  const int* sl;                  // [Vs] or null
  int* cand_local;                // [B][M]
  int* cand_global;               // [B][M] or null
  unsigned* keys;                 // ws [B][Vs]
  long long ld;
  int n, Vs, M;
};

// keys[b][j] for 4 columns a thread, grid (B, column blocks): coalesced and spread over the chip
__global__ void __launch_bounds__(256) k_cand_keys(CandArgs a) {
  const int b = blockIdx.x;
  for (int q = 0; q < 4; ++q) {
    const int j = (blockIdx.y * 4 + q) * 256 + threadIdx.x;
    if (j >= a.Vs) return;
    float v = -INFINITY;
    for (int d = 0; d < a.n; ++d) {
      const size_t r = (size_t)b * a.n + d;
      v = fmaxf(v, (float)__builtin_bit_cast(_Float16, a.logits[r * a.ld + j]) - a.lse[r]);
    }
    a.keys[(size_t)b * a.Vs + j] = order_key(v);
  }
}

// Radix select in three digits of the 32-bit key -- bits 31..20, 19..8, 7..0 (4096 / 4096 / 256
// bins): the wide first digit spreads the log-probabilities, whose top bits (sign and exponent)
// take only a few values, over many bins instead of serialising the histogram atomics on one.
// Each pass counts only the keys that match the digits chosen so far; the digit holding the M-th
// largest key is found by a workgroup scan over the bins (thread t owns bins 4t .. 4t+3 from the
// top).
__device__ void select_digit(const unsigned* keys, int Vs, unsigned prefix, unsigned pmask, int shift, int bins,
                             int* hist, int* scan, unsigned* s_prefix, int* s_rem) {
  const int t = threadIdx.x;
  for (int i = t; i < bins; i += CT) hist[i] = 0;
  __syncthreads();
  const unsigned dmask = (unsigned)bins - 1;
  for (int j = t; j < Vs; j += CT) {
    const unsigned k = keys[j];
    if ((k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & dmask], 1);
  }
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

__global__ void __launch_bounds__(CT) k_cand_select(CandArgs a) {
  __shared__ int hist[4096];
  __shared__ int scan[CT];
  __shared__ unsigned s_prefix;
  __shared__ int s_rem;
  const int b = blockIdx.x, t = threadIdx.x;
  const unsigned* keys = a.keys + (size_t)b * a.Vs;
  if (t == 0) { s_prefix = 0; s_rem = a.M; }
  __syncthreads();
  select_digit(keys, a.Vs, 0u, 0u, 20, 4096, hist, scan, &s_prefix, &s_rem);
  select_digit(keys, a.Vs, s_prefix, 0xFFF00000u, 8, 4096, hist, scan, &s_prefix, &s_rem);
  select_digit(keys, a.Vs, s_prefix, 0xFFFFFF00u, 0, 256, hist, scan, &s_prefix, &s_rem);
  const unsigned T = s_prefix;
  const int need = s_rem;   // ties at T that belong to the M (lowest columns first)
  // compaction in column order: thread t owns the contiguous columns [c0, c1)
  const int per = (a.Vs + CT - 1) / CT;
  const int c0 = min(t * per, a.Vs), c1 = min(c0 + per, a.Vs);
  int gt = 0, eq = 0;
  for (int j = c0; j < c1; ++j) {
    const unsigned k = keys[j];
    gt += k > T;
    eq += k == T;
  }
  int tot;
  const int eq_before = block_exscan(eq, scan, &tot);
  const int take_eq = min(max(need - eq_before, 0), eq);
  int out = block_exscan(gt + take_eq, scan, &tot);
  int eq_seen = 0;
  int* cl = a.cand_local + (size_t)b * a.M;
  int* cg = a.cand_global ? a.cand_global + (size_t)b * a.M : nullptr;
  for (int j = c0; j < c1; ++j) {
    const unsigned k = keys[j];
    bool take = k > T;
    if (k == T) take = eq_seen++ < take_eq;
    if (take) {
      cl[out] = j;
      if (cg) cg[out] = a.sl ? a.sl[j] : j;
      ++out;
    }
  }
}

}  // namespace

extern "C" {

int64_t cfh_cand_ws_bytes(int B, int Vs) {
  if (B < 0 || Vs < 0) return -1;
  return (int64_t)B * Vs * 4;
}

int cfh_cand_topm(const void* logits, long long ld, const float* lse, int B, int n, int Vs, int M, const int32_t* sl,
                  int32_t* cand_local, int32_t* cand_global, void* ws, void* stream) {
  if (B == 0) return CFH_OK;
  if (!logits || !lse || !cand_local || !ws || B < 0 || n < 1 || Vs < 1 || M < 1 || M > Vs || ld < Vs)
    return CFH_E_INVALID;
  CandArgs a = {(const unsigned short*)logits, lse, sl, cand_local, cand_global, (unsigned*)ws, ld, n, Vs, M};
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(k_cand_keys, dim3(B, (Vs + 1023) / 1024), dim3(256), 0, st, a);
  CFH_LAUNCH_CHECK();
  hipLaunchKernelGGL(k_cand_select, dim3(B), dim3(CT), 0, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

}  // extern "C"
