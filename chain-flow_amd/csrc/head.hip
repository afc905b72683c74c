// The draft head on MI355X: shortlisted lm_head (+ markov bias) with fused per-row log-softmax
// top-k, the batched (MFMA skinny-GEMM) head, the path-conditioned residual and the beam-search
// steps of the proposer.
//
// Reference semantics (cf/ = src/chain_flow/):
//   _head  = h.to(fp16) @ lm_w[sl].T -> fp16 logits      cf/vllm_plugin/flow_proposer.py:1021-1022, 739
//   _bias  = markov.w1(prev) @ markov.w2.weight[sl].T     :1024-1025, 740; cf/drafters/markov_flow.py:62-74
//   lp = log_softmax(logits.float()); topk(lp, W)         :1249-1250
//   _map   = sl[local]                                     :1027-1028
//   two-pass head, pass A: one GEMM over the B*K marginal hiddens, then per-row top-M
//                                                          :1142-1165
//   fused path residual (one baddbmm over live offsets, masked sum, LN -> Linear -> GELU -> Linear)
//                                                          cf/vllm_plugin/fused.py:25-37
//   _beam_chains / _beam_tree depth steps and backtrack    :1187-1332
//
// The heads read the rows of the target's lm_head in place through the int32 shortlist (a row
// gather), so no gathered copy of lm_w[sl] is needed.  The logits never have to reach HBM: each
// workgroup reduces its column block to per-row (max, sum-exp) and a local top-k, and a merge
// kernel combines the blocks into the row's log-sum-exp and top-k.
#include <limits.h>

#include "cfh_wide.h"

namespace {

constexpr int HW = 8;       // waves per head workgroup (one 16-row vocabulary tile per wave)
constexpr int HCOLS = HW * 16;
constexpr int HMAXM = 8;    // max activation rows of the in-place GEMV head
constexpr int KMAX = 16;    // max top-k
constexpr int PATH_CHUNK = 16;   // rows of one path-residual launch sequence (the GEMV's row limit)

// (value, index) order: larger value first, equal values by lower index.
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// Arg-best of (v, i) over the lanes of an aligned group of W lanes (W = 16 or 64), in every lane
// of the group.  `better` is a total order, so the result does not depend on the pairing.
template <int CTRL>
__device__ __forceinline__ void best_step(float& v, int& i) {
  const float ov = dpp_f32<CTRL>(v);
  const int oi = dpp_i32<CTRL>(i);
  if (better(ov, oi, v, i)) { v = ov; i = oi; }
}

template <int W>
__device__ __forceinline__ void group_best(float& v, int& i) {
  static_assert(W == 16 || W == 64, "group_best: 16 or 64 lanes");
  best_step<DPP_XOR1>(v, i);
  best_step<DPP_XOR2>(v, i);
  best_step<DPP_HMIRROR>(v, i);
  best_step<DPP_MIRROR>(v, i);
  if constexpr (W == 64) {
    float bv = readlane_f32(v, 0);
    int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
      const float rv = readlane_f32(v, r);
      const int ri = __builtin_amdgcn_readlane(i, r);
      if (better(rv, ri, bv, bi)) { bv = rv; bi = ri; }
    }
    v = bv;
    i = bi;
  }
}

// Per-thread sorted list of the best KMAX (value, index) pairs seen.
struct TopList {
  float v[KMAX];
  int i[KMAX];
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int q = 0; q < KMAX; ++q) { v[q] = -INFINITY; i[q] = INT_MAX; }
  }
  __device__ __forceinline__ void push(float x, int ix) {
    if (!better(x, ix, v[KMAX - 1], i[KMAX - 1])) return;
    v[KMAX - 1] = x;
    i[KMAX - 1] = ix;
#pragma unroll
    for (int q = KMAX - 1; q > 0; --q) {
      if (better(v[q], i[q], v[q - 1], i[q - 1])) {
        const float tv = v[q]; v[q] = v[q - 1]; v[q - 1] = tv;
        const int ti = i[q]; i[q] = i[q - 1]; i[q - 1] = ti;
      }
    }
  }
  __device__ __forceinline__ void pop() {
#pragma unroll
    for (int q = 0; q < KMAX - 1; ++q) { v[q] = v[q + 1]; i[q] = i[q + 1]; }
    v[KMAX - 1] = -INFINITY;
    i[KMAX - 1] = INT_MAX;
  }
};

// k rounds of a block-wide arg-best over the heads of every thread's TopList; thread 0 receives
// the winners in order through emit(r, v, i).  Uses red_v/red_i[nwaves].
template <typename Emit>
__device__ void block_select(TopList& L, int k, float* red_v, int* red_i, Emit emit) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  for (int r = 0; r < k; ++r) {
    float bv = L.v[0];
    int bi = L.i[0];
    group_best<64>(bv, bi);
    __syncthreads();
    if (lane == 0) { red_v[wave] = bv; red_i[wave] = bi; }
    __syncthreads();
    bv = red_v[0];
    bi = red_i[0];
    for (int w = 1; w < nw; ++w)
      if (better(red_v[w], red_i[w], bv, bi)) { bv = red_v[w]; bi = red_i[w]; }
    if (L.i[0] == bi && bi != INT_MAX) L.pop();   // the owner of the winner advances
    if (threadIdx.x == 0) emit(r, bv, bi);
  }
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t = fmaxf(t, red[w]);
  return t;
}

// Candidate sets written by the head kernels: for row m and column block b,
//   cv/ci [(m * nsets + b) * k + r]  the block's r-th best (fp16/bf16-rounded logit, column)
//   cs    [(m * nsets + b) * 2]      the block's (max, sum of exp(logit - max))
struct Cands {
  float* cv;
  int* ci;
  float* cs;
  int nsets, k;
};

__host__ __device__ __forceinline__ size_t cand_bytes(int M, int nsets, int k) {
  return (size_t)M * nsets * ((size_t)k * 8 + 8);
}

__device__ __forceinline__ Cands carve_cands(void* ws, int M, int nsets, int k) {
  Cands c;
  c.cv = (float*)ws;
  c.ci = (int*)(c.cv + (size_t)M * nsets * k);
  c.cs = (float*)(c.ci + (size_t)M * nsets * k);
  c.nsets = nsets;
  c.k = k;
  return c;
}

// ---------------------------------------------------------------------------- GEMV head
struct HeadArgs {
  const h16* h;        // [M][d]
  const h16* W;        // [V][d]
  const int* sl;       // [n] shortlist (global row ids) or null: rows 0..n-1
  const h16* a;        // markov A: [M][r] rows, or the w1 table when a_ids is set
  const int* a_ids;    // row ids into a (a_ids[m * a_ids_stride]), or null
  const h16* W2;       // [V][r] markov w2 or null
  h16* logits;         // [M][n] or null
  void* ws;            // candidate sets (null: logits only)
  int M, d, n, r, a_ids_stride, k, nsets;
  // request groups (grid.y): group g scores its own M rows (h + g M d) against its own n rows
  // sl + g sl_stride; its candidates are rows g M .. g M + M - 1 of the workspace (G M rows)
  int groups;
  long long sl_stride;
};

// Packed head image (cfh_head_pack): the shortlisted rows of W, then those of the markov w2, in
// the MFMA fragment order -- fragment (tile t, k-step s) = 1 KiB at (t * K/32 + s) * 64 vectors,
// lane l holding row sl[16 t + l % 16], columns 32 s + 8 (l / 16) .. +7.  Columns past n repeat
// the last shortlisted row.
__host__ __device__ __forceinline__ size_t head_packed_w_bytes(int n, int d) {
  return (size_t)((n + 15) / 16) * 16 * d * 2;
}

// One wave per 16-row vocabulary tile, HW tiles per workgroup.  Each lane streams its vocabulary
// row in place (row-major lm_head, 16 bytes per k-step) against the M activation rows in LDS with
// v_mfma_f32_16x16x32_f16; the markov bias is a second, rank-r MFMA stream over w2.  Epilogue:
// logit = fp16(fp16(h.W) + fp16(A.W2)); per row, the block's (max, sum-exp) and top-k.
//
// PACKED: W and W2 point at a cfh_head_pack image instead (same results): each wave then streams
// one contiguous 1 KiB fragment per k-step rather than 16 rows 64 bytes at a time.
template <bool PACKED>
__global__ void __launch_bounds__(HW * 64) k_head(HeadArgs a) {
  extern __shared__ __align__(16) h16 sm[];
  __shared__ float Lt[HMAXM][HCOLS];
  const int grp = blockIdx.y;
  if (grp > 0) {
    a.h += (size_t)grp * a.M * a.d;
    if (a.sl) a.sl += (size_t)grp * a.sl_stride;
    if (a.a_ids) a.a_ids += (size_t)grp * a.M * a.a_ids_stride;
    else if (a.a) a.a += (size_t)grp * a.M * a.r;
    if (a.logits) a.logits += (size_t)grp * a.M * a.n;
  }
  const int ldh = a.d + 8, ldm = a.r + 8;
  h16* Ah = sm;
  h16* Am = sm + a.M * ldh;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * HW + wave;
  const int ntiles = (a.n + 15) / 16;
  const int j = t * 16 + (lane & 15);
  const bool colv = (t < ntiles) && (j < a.n);
  const int jc = colv ? j : a.n - 1;                 // padding lanes load a valid row
  const size_t row = PACKED ? 0 : (a.sl ? (size_t)a.sl[jc] : (size_t)jc);
  const size_t tp = (size_t)min(t, ntiles - 1);      // packed: padding waves stream the last tile
  // the markov fragments (r/32 per lane) are put in flight first: they are few and are used last
  TileStream<PF, PACKED ? 64 : 4, PACKED> tm;
  if (a.W2) {
    if constexpr (PACKED) tm.begin((const h16x8*)a.W2 + tp * (a.r / 32) * 64, a.r / 32);
    else tm.begin((const h16x8*)(a.W2 + row * a.r + 8 * (lane >> 4)), a.r / 32);
  }
  TileStream<PF, PACKED ? 64 : 4, PACKED> ts;
  if constexpr (PACKED) ts.begin((const h16x8*)a.W + tp * (a.d / 32) * 64, a.d / 32);
  else ts.begin((const h16x8*)(a.W + row * a.d + 8 * (lane >> 4)), a.d / 32);
  const int nh = a.d / 8;
  batched_copy(a.M * nh,
               [&](int idx) {
                 const int i = idx / nh, kk = (idx - i * nh) * 8;
                 return *(const h16x8*)(a.h + (size_t)i * a.d + kk);
               },
               [&](int idx, h16x8 v) {
                 const int i = idx / nh, kk = (idx - i * nh) * 8;
                 *(h16x8*)(Ah + i * ldh + kk) = v;
               });
  if (a.W2) {
    const int nm = a.r / 8;
    batched_copy(a.M * nm,
                 [&](int idx) {
                   const int i = idx / nm, kk = (idx - i * nm) * 8;
                   const size_t src = a.a_ids ? (size_t)max(a.a_ids[i * a.a_ids_stride], 0) : (size_t)i;
                   return *(const h16x8*)(a.a + src * a.r + kk);
                 },
                 [&](int idx, h16x8 v) {
                   const int i = idx / nm, kk = (idx - i * nm) * 8;
                   *(h16x8*)(Am + i * ldm + kk) = v;
                 });
  }
  __syncthreads();
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = ts.run(Ah, ldh, a.M, acc);
  f32x4 accm = {0.f, 0.f, 0.f, 0.f};
  if (a.W2) accm = tm.run(Am, ldm, a.M, accm);
  const int rbase = 4 * (lane >> 4);
  const int c = wave * 16 + (lane & 15);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rr = rbase + q;
    if (rr < a.M) {
      const float v = a.W2 ? r16(r16(acc[q]) + r16(accm[q])) : r16(acc[q]);
      if (a.logits && colv) a.logits[(size_t)rr * a.n + j] = (h16)v;
      Lt[rr][c] = colv ? v : -INFINITY;
    }
  }
  if (!a.ws) return;
  __syncthreads();
  if (wave >= a.M) return;
  // wave `wave` reduces row `wave` of this block's HCOLS columns
  const Cands cd = carve_cands(a.ws, a.M * max(a.groups, 1), a.nsets, a.k);
  const int m = wave;
  const int c0 = blockIdx.x * HCOLS + lane, c1 = c0 + 64;
  float x0 = Lt[m][lane], x1 = Lt[m][lane + 64];
  int i0 = x0 == -INFINITY ? INT_MAX : c0, i1 = x1 == -INFINITY ? INT_MAX : c1;
  const float mx = wave_max(fmaxf(x0, x1));
  const float se = mx == -INFINITY ? 0.f : wave_sum(expf(x0 - mx) + expf(x1 - mx));
  if (better(x1, i1, x0, i0)) {
    const float tv = x0; x0 = x1; x1 = tv;
    const int ti = i0; i0 = i1; i1 = ti;
  }
  const size_t base = ((size_t)grp * a.M + m) * a.nsets + blockIdx.x;
  for (int r = 0; r < a.k; ++r) {
    float bv = x0;
    int bi = i0;
    group_best<64>(bv, bi);
    if (i0 == bi && bi != INT_MAX) { x0 = x1; i0 = i1; x1 = -INFINITY; i1 = INT_MAX; }
    if (lane == 0) { cd.cv[base * a.k + r] = bv; cd.ci[base * a.k + r] = bi; }
  }
  if (lane == 0) { cd.cs[base * 2] = mx; cd.cs[base * 2 + 1] = se; }
}

// ---------------------------------------------------------------------------- merge
// One workgroup per row: log-sum-exp from the blocks' (max, sum-exp) and the top-k over the
// blocks' candidates.  vals = logit - lse, ids = column (-1 / -inf past the valid columns).
struct MergeArgs {
  const void* ws;
  int M, nsets, k;
  float* vals;
  int* ids;
  float* lse;
};

constexpr int MT_THREADS = 256;
constexpr int MBATCH = 8;

__global__ void __launch_bounds__(MT_THREADS) k_topk_merge(MergeArgs a) {
  __shared__ float red[MT_THREADS / 64];
  __shared__ float red_v[MT_THREADS / 64];
  __shared__ int red_i[MT_THREADS / 64];
  const Cands cd = carve_cands((void*)a.ws, a.M, a.nsets, a.k);
  const int m = blockIdx.x;
  const float* cs = cd.cs + (size_t)m * a.nsets * 2;
  float mx = -INFINITY;
  for (int b = threadIdx.x; b < a.nsets; b += blockDim.x) mx = fmaxf(mx, cs[b * 2]);
  mx = block_max(mx, red);
  float se = 0.f;
  for (int b = threadIdx.x; b < a.nsets; b += blockDim.x) {
    const float s = cs[b * 2 + 1];
    if (s > 0.f) se += s * expf(cs[b * 2] - mx);
  }
  se = block_sum(se, red);
  const float lse = mx + logf(se);
  if (threadIdx.x == 0 && a.lse) a.lse[m] = lse;
  const int total = a.nsets * a.k;
  const float* cv = cd.cv + (size_t)m * total;
  const int* ci = cd.ci + (size_t)m * total;
  TopList L;
  L.init();
  for (int base = 0; base < total; base += MBATCH * MT_THREADS) {
    float v[MBATCH];
    int ix[MBATCH];
#pragma unroll
    for (int q = 0; q < MBATCH; ++q) {
      const int e = base + q * MT_THREADS + threadIdx.x;
      v[q] = e < total ? cv[e] : -INFINITY;
      ix[q] = e < total ? ci[e] : INT_MAX;
    }
#pragma unroll
    for (int q = 0; q < MBATCH; ++q) L.push(v[q], ix[q]);
  }
  float* vals = a.vals + (size_t)m * a.k;
  int* ids = a.ids + (size_t)m * a.k;
  block_select(L, a.k, red_v, red_i, [&](int r, float bv, int bi) {
    const bool ok = bi != INT_MAX;
    vals[r] = ok ? bv - lse : -INFINITY;
    ids[r] = ok ? bi : -1;
  });
}

// The same merge with one wave per row and no workgroup barriers, for rows whose candidates fit in
// LDS (nsets * k * 8 bytes <= MW_LDS): every block's list is sorted best first, so the row's top-k
// is a k-way merge of the lists.  The wave stages the row's lists in LDS; lane l caches the heads
// of the blocks b = l + 64 s (s < S); each round is a lane argmax over S heads, a wave argmax (DPP),
// and the winning lane moves to its list's next entry.  Same results as k_topk_merge.
constexpr int MW_LDS = 64 * 1024;

// Row m by one wave, its lists staged at sv (nsets k floats, then as many ints).
template <int S>
__device__ void merge_row(const MergeArgs& a, int m, float* sv) {
  const int lane = threadIdx.x & 63;
  const Cands cd = carve_cands((void*)a.ws, a.M, a.nsets, a.k);
  const int k = a.k, total = a.nsets * k;
  int* si = (int*)(sv + total);
  const float* cv = cd.cv + (size_t)m * total;
  const int* ci = cd.ci + (size_t)m * total;
  // the lane's blocks' (max, sum-exp) first: loads complete in issue order, so the log-sum-exp
  // below does not wait for the staging loads
  const float2* cs = (const float2*)(cd.cs + (size_t)m * a.nsets * 2);
  float2 cq[S];
#pragma unroll
  for (int q = 0; q < S; ++q) {
    const int b = lane + 64 * q;
    cq[q] = b < a.nsets ? cs[b] : make_float2(-INFINITY, 0.f);
  }
  // staging: batches of 8 loads a lane issued before their LDS writes, 16 bytes each when the
  // row's lists start 16-byte aligned (total % 4 == 0)
  if ((total & 3) == 0) {
    const int nv = total / 4;
    for (int e0 = lane; e0 < nv; e0 += 64 * 8) {
      // loads unconditional (index clamped; the surplus is never stored), so the batch stays in
      // registers: a conditionally written array would live in scratch memory
      uint4 tv[8], ti[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = min(e0 + 64 * j, nv - 1);
        tv[j] = ((const uint4*)cv)[e];
        ti[j] = ((const uint4*)ci)[e];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = e0 + 64 * j;
        if (e < nv) {
          ((uint4*)sv)[e] = tv[j];
          ((uint4*)si)[e] = ti[j];
        }
      }
    }
  } else {
    for (int e0 = lane; e0 < total; e0 += 64 * 8) {
      float tv[8];
      int ti[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = min(e0 + 64 * j, total - 1);
        tv[j] = cv[e];
        ti[j] = ci[e];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = e0 + 64 * j;
        if (e < total) { sv[e] = tv[j]; si[e] = ti[j]; }
      }
    }
  }
  // log-sum-exp over the blocks' (max, sum-exp)
  float mx = -INFINITY;
#pragma unroll
  for (int q = 0; q < S; ++q) mx = fmaxf(mx, cq[q].x);
  mx = wave_max(mx);
  float se = 0.f;
#pragma unroll
  for (int q = 0; q < S; ++q)
    if (cq[q].y > 0.f) se += cq[q].y * expf(cq[q].x - mx);
  se = wave_sum(se);
  const float lse = mx + logf(se);
  if (lane == 0 && a.lse) a.lse[m] = lse;
  // the staged lists are read by other lanes of this wave: LDS accesses of one wave complete in
  // order, the fence keeps the compiler from moving the reads above the writes
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  float hv[S];
  int hi[S], pos[S];
#pragma unroll
  for (int q = 0; q < S; ++q) {
    const int b = lane + 64 * q;
    pos[q] = 0;
    hv[q] = b < a.nsets ? sv[b * k] : -INFINITY;
    hi[q] = b < a.nsets ? si[b * k] : INT_MAX;
  }
  float* vals = a.vals + (size_t)m * k;
  int* ids = a.ids + (size_t)m * k;
  for (int r = 0; r < k; ++r) {
    float bv = hv[0];
    int bi = hi[0], bq = 0;
#pragma unroll
    for (int q = 1; q < S; ++q)
      if (better(hv[q], hi[q], bv, bi)) { bv = hv[q]; bi = hi[q]; bq = q; }
    float gv = bv;
    int gi = bi;
    group_best<64>(gv, gi);
    if (bi == gi && gi != INT_MAX) {                     // the owner of the winner advances
#pragma unroll
      for (int q = 0; q < S; ++q)
        if (q == bq) {
          const int b = lane + 64 * q;
          const int p = ++pos[q];
          hv[q] = p < k ? sv[b * k + p] : -INFINITY;
          hi[q] = p < k ? si[b * k + p] : INT_MAX;
        }
    }
    if (lane == 0) {
      const bool ok = gi != INT_MAX;
      vals[r] = ok ? gv - lse : -INFINITY;
      ids[r] = ok ? gi : -1;
    }
  }
}

template <int S>
__global__ void __launch_bounds__(256) k_merge_wave(MergeArgs a) {
  extern __shared__ __align__(16) float mw[];
  const int wave = threadIdx.x >> 6;
  const int m = blockIdx.x * (blockDim.x >> 6) + wave;
  if (m >= a.M) return;                                  // (no workgroup barrier below)
  merge_row<S>(a, m, mw + (size_t)wave * a.nsets * a.k * 2);
}

// ---------------------------------------------------------------------------- row top-k
// Standalone per-row log-softmax top-k of fp16 logits [M][n] (one workgroup per row): every
// thread loads its columns in batches (all loads of a batch in flight together), keeps an online
// (max, sum-exp) and a sorted top list, then the block selects the k best.
struct TopkArgs {
  const h16* logits;   // [M][ld]
  int ld, M, n, k;
  float* vals;         // [M][k] logit - logsumexp
  int* ids;            // [M][k]
  float* lse;          // [M] or null
};

constexpr int TK_THREADS = 1024;

__global__ void __launch_bounds__(TK_THREADS) k_topk(TopkArgs a) {
  __shared__ float red[TK_THREADS / 64];
  __shared__ float red_v[TK_THREADS / 64];
  __shared__ int red_i[TK_THREADS / 64];
  const int row = blockIdx.x;
  const h16* L = a.logits + (size_t)row * a.ld;
  TopList T;
  T.init();
  float m = -INFINITY, s = 0.f;
  for (int base = 0; base < a.n; base += MBATCH * TK_THREADS) {
    float v[MBATCH];
#pragma unroll
    for (int q = 0; q < MBATCH; ++q) {
      const int e = base + q * TK_THREADS + threadIdx.x;
      v[q] = e < a.n ? (float)L[e] : -INFINITY;
    }
    float bm = m;
#pragma unroll
    for (int q = 0; q < MBATCH; ++q) bm = fmaxf(bm, v[q]);
    if (bm != -INFINITY) {
      s = (m == -INFINITY ? 0.f : s * expf(m - bm));
#pragma unroll
      for (int q = 0; q < MBATCH; ++q) s += expf(v[q] - bm);
      m = bm;
    }
#pragma unroll
    for (int q = 0; q < MBATCH; ++q) {
      const int e = base + q * TK_THREADS + threadIdx.x;
      if (e < a.n) T.push(v[q], e);
    }
  }
  const float mx = block_max(m, red);
  const float se = block_sum(m == -INFINITY ? 0.f : s * expf(m - mx), red);
  const float lse = mx + logf(se);
  if (threadIdx.x == 0 && a.lse) a.lse[row] = lse;
  float* vals = a.vals + (size_t)row * a.k;
  int* ids = a.ids + (size_t)row * a.k;
  block_select(T, a.k, red_v, red_i, [&](int r, float bv, int bi) {
    const bool ok = bi != INT_MAX;
    vals[r] = ok ? bv - lse : -INFINITY;
    ids[r] = ok ? bi : -1;
  });
}

// ---------------------------------------------------------------------------- MFMA GEMM head
// Batched head (M up to 256 rows, bf16, or fp16 with the markov bias): a workgroup of GW waves
// owns GW*NT*16 vocabulary rows; each wave streams NT row tiles (in place through the shortlist,
// or from the packed image with non-temporal loads) and multiplies every B fragment against the MT
// 16-row tiles of the activations (v_mfma_f32_16x16x32_bf16 / _f16), so one weight byte feeds
// 16*MT rows.  The activations pass through LDS in 128-column chunks, double-buffered: the
// next chunk's loads are in flight while the current one is multiplied.  The weight fragments
// alternate between two register sets by chunk parity, so each chunk's weights are requested a
// whole chunk of multiplies ahead.  Two waves a SIMD (GW = 8) keep the accumulators and both sets
// in registers, and one wave's multiplies run while the other waits.  PK: the weights come from a
// cfh_head_pack image, whose 16-row x 32-column fragments are the MFMA B operands in lane order,
// so every wave load is 1 KB contiguous (in place: 16 rows x 64 bytes).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// A weight fragment load of the GEMM heads.  From a packed image it is non-temporal, since each
// byte is read once per call (measured on the 62,642-row, d=4096 stream: 6.2 against 5.5 TB/s
// with the default policy); in place each lane reads 16 bytes of a row whose other bytes the next
// k-steps read, so the lines should stay in L2 (non-temporal there fetched 663 MB for 515).
template <bool PK>
__device__ __forceinline__ bf16x8 wload(const bf16x8* p) {
  if constexpr (PK) return __builtin_bit_cast(bf16x8, __builtin_nontemporal_load((const h16x8*)p));
  else return *p;
}

constexpr int GPF = 4;            // k-steps per LDS chunk
// M <= 160 rows: 2 column tiles per wave, all 10 row tiles in each wave.  (Splitting the row tiles
// over 2 waves with 4 column tiles each -- an x operand read feeding 4 MFMAs, twice the weights in
// flight -- needs more than the 256 registers a wave has at 2 waves per SIMD: it spills.)
constexpr int GEMM160_NT = 2, GEMM160_MS = 1;
constexpr int GKC = 32 * GPF;     // 128 columns per chunk: a row is 16 slots of 16 bytes

struct GemmArgs {
  const uint16_t* x;   // [M][d] bf16 (F16: fp16)
  const uint16_t* W;   // [V][d] bf16 (F16: fp16)
  const int* sl;
  const uint16_t* bias;  // F16 only: [M][n] fp16 added before the last rounding, or null
  uint16_t* logits;    // [M][n] bf16 (F16: fp16) or null
  void* ws;
  int M, d, n, k, nsets;   // k = 0: logits only, no top-k
};

// The 16-bit logit of a GEMM accumulator: bf16(acc), or fp16(acc) -- fp16(fp16(acc) + bias) with a
// bias, the rounding points of the GEMV head's fp16(fp16(h.W) + fp16(A.W2)).
template <bool F16>
__device__ __forceinline__ uint16_t gemm_logit(float acc, const uint16_t* bias) {
  if constexpr (F16) {
    h16 v = (h16)acc;
    if (bias) v = (h16)((float)v + (float)__builtin_bit_cast(h16, *bias));
    return __builtin_bit_cast(uint16_t, v);
  } else {
    return __builtin_bit_cast(uint16_t, (__bf16)acc);
  }
}

// The value of a 16-bit logit's bit pattern.
template <bool F16>
__device__ __forceinline__ float gemm_value(unsigned b) {
  if constexpr (F16) return (float)__builtin_bit_cast(h16, (uint16_t)b);
  else return __uint_as_float(b << 16);
}

// median of three (one v_med3_u32)
__device__ __forceinline__ unsigned umed3(unsigned a, unsigned b, unsigned c) { return max(min(a, b), min(max(a, b), c)); }

// Epilogue of the GEMM heads.  The wave's accumulators -- row tiles rt0 .. rt0+MTW-1, columns
// c0 .. c0+NT*16-1 of the block's COLS -- become 16-bit logits (gemm_logit), written to a.logits and
// parked in LDS as [rows][COLS + 8] over the operand buffers (the caller has passed a barrier after
// its last operand read).  Then one 16-lane group a row ranks the block's COLS columns: lane l holds
// columns l*CPL .. l*CPL+CPL-1 as 32-bit keys (order-preserving 16-bit logit << 16 | 0xFFFF -
// column), so one integer max picks the larger logit and, on a tie, the lower column.  Key 0 = no
// column.  The block's top-k and (max, sum of exp) go to the candidate lists for the merge.
template <int MTW, int NT, int COLS, int NTHR, int ROWS, bool F16>
__device__ __forceinline__ void gemm_finish(const GemmArgs& a, const f32x4 (&acc)[MTW][NT], uint16_t* lg, int rt0,
                                            int c0) {
  constexpr int LST = COLS + 8, CPL = COLS / 16;
  static_assert(CPL % 8 == 0, "a lane's columns are read as 16-byte vectors");
  const int lane = threadIdx.x & 63;
  {
    // to LDS without branches (rows past M and columns past the shortlist hold values nothing
    // reads; the bias of such an element is read at a clamped, valid position), then to a.logits
    // when asked for: per-element branches here cost more than the stores
    const int g = lane >> 4, col = lane & 15;
    const bool bias = F16 && a.bias;
#pragma unroll
    for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = (rt0 + mt) * 16 + 4 * g + q;
          const int c = c0 + t * 16 + col;
          const int j = blockIdx.x * COLS + c;
          lg[r * LST + c] = gemm_logit<F16>(acc[mt][t][q],
                                            bias ? a.bias + (size_t)min(r, a.M - 1) * a.n + min(j, a.n - 1) : nullptr);
        }
    if (a.logits) {
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int r = (rt0 + mt) * 16 + 4 * g + q;
            const int c = c0 + t * 16 + col;
            const int j = blockIdx.x * COLS + c;
            if (r < a.M && j < a.n) a.logits[(size_t)r * a.n + j] = lg[r * LST + c];
          }
    }
  }
  if (a.k == 0) return;      // logits only
  lds_barrier();
  const Cands cd = carve_cands(a.ws, a.M, a.nsets, a.k);
  const int col = lane & 15;
  // A 16-lane group ranks RB rows together (rows r0 + b*NGR), their independent chains
  // interleaved.  Each lane keeps the four largest of its CPL keys below fl (its last key taken;
  // initially above every key) in q0 >= q1 >= q2 >= q3; a round takes the group's largest q0
  // (4 DPP steps) and the winning lane shifts its four up.  A lane refills from LDS only when it
  // wins a fifth time: a row's top k rarely takes more than four of one lane's sixteen columns.
  constexpr int NGR = NTHR / 16, RPG = (ROWS + NGR - 1) / NGR, NIT = (RPG + 4) / 5, RB = (RPG + NIT - 1) / NIT;
  const int nrem = a.n - (int)blockIdx.x * COLS - col * CPL;   // the lane's columns: i < nrem
  const bool whole = (int)(blockIdx.x + 1) * COLS <= a.n;      // every column of the block is live
  // the four largest keys below lim of the lane's columns of row r (keys past the shortlist: 0).
  // Arithmetic throughout: compares here would each hold an SGPR-pair mask.  A key enters the
  // sorted four with one max and three medians of three (v_med3_u32).
  auto lane_top4 = [&](int r, unsigned lim, bool limited, bool masked, unsigned (&q)[4]) {
    q[0] = q[1] = q[2] = q[3] = 0u;
#pragma unroll
    for (int h = 0; h < CPL / 8; ++h) {
      const uint4 u = *(const uint4*)(lg + r * LST + col * CPL + h * 8);
      const unsigned w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        // two logits a word: -0 ranks as +0 (clears only its sign), then order-preserving bits
        unsigned x = w4[w];
        x &= 0x7FFF7FFFu | ((x & 0x7FFF7FFFu) + 0x7FFF7FFFu);
        x ^= 0x80008000u | (((x >> 15) & 0x00010001u) * 0x7FFFu);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int i = h * 8 + w * 2 + e, c = col * CPL + i;
          unsigned t = (e ? (x & 0xFFFF0000u) : (x << 16)) | (0xFFFFu - (unsigned)c);
          if (masked) t &= 0u - ((unsigned)(i - nrem) >> 31);
          if (limited) t = t < lim ? t : 0u;
          const unsigned n0 = max(q[0], t), n1 = umed3(q[0], q[1], t), n2 = umed3(q[1], q[2], t),
                         n3 = umed3(q[2], q[3], t);
          q[0] = n0; q[1] = n1; q[2] = n2; q[3] = n3;
        }
      }
    }
  };
  // The winners' keys and each row's (max, sum-exp) are staged in LDS after the logits, written by
  // every lane of the group (the same value: no branch), rows past M into a dummy slot ROWS; one
  // pass at the end decodes the keys into (value, column) and copies them out.  Branches inside a
  // round would split it into blocks the compiler cannot interleave across rows (and copy the
  // rows' lists at each).
  auto key_value = [](unsigned key) -> float {
    const unsigned o = key >> 16;
    return key ? gemm_value<F16>((o & 0x8000u) ? (o & 0x7FFFu) : (~o & 0xFFFFu)) : -INFINITY;
  };
  unsigned* cstk = (unsigned*)(lg + ROWS * LST);
  float* cstm = (float*)(cstk + (ROWS + 1) * KMAX);
  float* csts = cstm + (ROWS + 1);
  for (int r0 = threadIdx.x >> 4; r0 < a.M; r0 += NGR * RB) {
    unsigned q[RB][4], fl[RB], k0[RB];
    bool full[RB];
    int slot[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const int r = r0 + b * NGR;
      slot[b] = r < a.M ? r : ROWS;
      if (r >= a.M) q[b][0] = q[b][1] = q[b][2] = q[b][3] = 0u;
      else if (whole) lane_top4(r, 0u, false, false, q[b]);
      else lane_top4(r, 0u, false, true, q[b]);
      fl[b] = 0xFFFFFFFFu;
      full[b] = q[b][3] != 0u;
    }
    for (int rr = 0; rr < a.k; ++rr) {
      unsigned m[RB];
#pragma unroll
      for (int b = 0; b < RB; ++b) m[b] = max(q[b][0], (unsigned)dpp_i32<DPP_XOR1>((int)q[b][0]));
#pragma unroll
      for (int b = 0; b < RB; ++b) m[b] = max(m[b], (unsigned)dpp_i32<DPP_XOR2>((int)m[b]));
#pragma unroll
      for (int b = 0; b < RB; ++b) m[b] = max(m[b], (unsigned)dpp_i32<DPP_HMIRROR>((int)m[b]));
#pragma unroll
      for (int b = 0; b < RB; ++b) m[b] = max(m[b], (unsigned)dpp_i32<DPP_MIRROR>((int)m[b]));
      bool need[RB], any = false;
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const bool win = m[b] != 0u && q[b][0] == m[b];
        fl[b] = win ? m[b] : fl[b];
        q[b][0] = win ? q[b][1] : q[b][0];
        q[b][1] = win ? q[b][2] : q[b][1];
        q[b][2] = win ? q[b][3] : q[b][2];
        q[b][3] = win ? 0u : q[b][3];
        need[b] = win && full[b] && q[b][0] == 0u;
        any |= need[b];
        k0[b] = rr == 0 ? m[b] : k0[b];
        cstk[slot[b] * KMAX + rr] = m[b];
      }
      if (__builtin_amdgcn_ballot_w64(any)) {      // rare: a lane won a fifth time
#pragma unroll
        for (int b = 0; b < RB; ++b)
          if (need[b]) {
            lane_top4(r0 + b * NGR, fl[b], true, true, q[b]);
            full[b] = q[b][3] != 0u;
          }
      }
    }
    // the row's sum of exp(logit - max), from the logits parked in LDS (hardware exp2)
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      const int r = r0 + b * NGR;
      const float mx = key_value(k0[b]);
      float se = 0.f;
      if (r < a.M && mx != -INFINITY) {
        const float nm = -mx * 1.4426950408889634f;
#pragma unroll
        for (int h = 0; h < CPL / 8; ++h) {
          const uint4 u = *(const uint4*)(lg + r * LST + col * CPL + h * 8);
          const unsigned w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int i = h * 8 + e;
            const unsigned v = (w4[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
            if (i < nrem) se += __builtin_amdgcn_exp2f(fmaf(gemm_value<F16>(v), 1.4426950408889634f, nm));
          }
        }
      }
      se = row_sum(se);
      cstm[slot[b]] = mx;
      csts[slot[b]] = se;
    }
  }
  lds_barrier();
  for (int i = threadIdx.x; i < a.M * a.k; i += NTHR) {
    const int r = i / a.k, rr = i - r * a.k;
    const size_t base = ((size_t)r * a.nsets + blockIdx.x) * a.k + rr;
    const unsigned key = cstk[r * KMAX + rr];
    cd.cv[base] = key_value(key);
    cd.ci[base] = key ? (int)blockIdx.x * COLS + (int)(0xFFFFu - (key & 0xFFFFu)) : INT_MAX;
  }
  for (int r = threadIdx.x; r < a.M; r += NTHR) {
    const size_t base = (size_t)r * a.nsets + blockIdx.x;
    cd.cs[base * 2] = cstm[r];
    cd.cs[base * 2 + 1] = csts[r];
  }
}

// MS: the MT row tiles are split over MS waves that share the same NT column tiles (the waves of a
// workgroup are NG = GW / MS column groups times MS row groups), so each x operand read from LDS
// feeds NT MFMAs and each wave keeps NT tiles of weight fragments in flight.
template <int MT, int NT, int GW, bool PK, bool F16, int MS>
__global__ void __launch_bounds__(GW * 64) k_head_gemm(GemmArgs a) {
  // [2][MT*16][GKC], each row's 16-byte slots XOR-swizzled by the row's low 4 bits: the 16 rows
  // an MFMA operand read touches then fall on 16 different bank groups
  extern __shared__ __align__(16) uint16_t xs[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  constexpr int ROWS = MT * 16, NG = GW / MS, MTW = MT / MS;
  static_assert(NG * MS == GW && MTW * MS == MT, "the row tiles and waves must split evenly");
  const int ng = wave % NG, mh = wave / NG;
  const int tile0 = (blockIdx.x * NG + ng) * NT;
  // fragment (tile, k-step s) of lane: wp[t][s * KS]; tiles past the shortlist re-read its last one
  constexpr int KS = PK ? 64 : 4;
  const bf16x8* wp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if constexpr (PK) {
      const int tile = min(tile0 + t, (a.n + 15) / 16 - 1);
      wp[t] = (const bf16x8*)a.W + (size_t)tile * (a.d / 32) * 64 + lane;
    } else {
      const int j = (tile0 + t) * 16 + (lane & 15);
      const int jc = j < a.n ? j : a.n - 1;
      const size_t row = a.sl ? (size_t)a.sl[jc] : (size_t)jc;
      wp[t] = (const bf16x8*)(a.W + row * a.d) + (lane >> 4);
    }
  }
  const int nchunks = a.d / GKC;
  // two register sets of weight fragments, for even and odd chunks: while chunk c is multiplied
  // from one set, the other holds chunk c+1 in flight, and each k-step's fragments are reloaded
  // with chunk c+2's right after their last multiply, in the same registers (nothing is copied at
  // the loop edge, so no wait drains the loads)
  bf16x8 bqa[GPF][NT], bqb[GPF][NT];
#pragma unroll
  for (int p = 0; p < GPF; ++p)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      bqa[p][t] = wload<PK>(wp[t] + p * KS);
      bqb[p][t] = wload<PK>(wp[t] + (min(1, nchunks - 1) * GPF + p) * KS);
    }
  // x chunk: ROWS x 16 vectors of 8, XV a thread (vector idx = row*16 + v); branch-free, rows past
  // M repeat row M-1 (their products are never read), so the wait counts before the multiplies
  // count these loads exactly and leave the weight loads in flight
  constexpr int XV = ROWS * 16 / (GW * 64);
  static_assert(XV * GW * 64 == ROWS * 16, "x chunk must split evenly over the workgroup");
  auto load_x = [&](int c, bf16x8* xr) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int idx = threadIdx.x + i * GW * 64;
      xr[i] = *(const bf16x8*)(a.x + (size_t)min(idx >> 4, a.M - 1) * a.d + c * GKC + (idx & 15) * 8);
    }
  };
  auto store_x = [&](int buf, const bf16x8* xr) {
    uint16_t* xb = xs + (size_t)buf * ROWS * GKC;
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int idx = threadIdx.x + i * GW * 64;
      const int r = idx >> 4;
      *(bf16x8*)(xb + r * GKC + ((idx & 15) ^ (r & 15)) * 8) = xr[i];
    }
  };
  {
    bf16x8 xr[XV];
    load_x(0, xr);
    store_x(0, xr);
  }
  lds_barrier();
  f32x4 acc[MTW][NT];
#pragma unroll
  for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[mt][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  auto step = [&](int c, bf16x8 (&bq)[GPF][NT]) {
    // chunks past the end are clamped to the last: the x re-read lands in the idle LDS buffer,
    // which nothing reads again, and the weight re-read is never multiplied
    bf16x8 xr[XV];
    load_x(min(c + 1, nchunks - 1), xr);
    const int cw = min(c + 2, nchunks - 1);
    const uint16_t* xb = xs + (size_t)(c & 1) * ROWS * GKC + (size_t)(mh * MTW * 16 + (lane & 15)) * GKC;
#pragma unroll
    for (int p = 0; p < GPF; ++p) {
      const int slot = (p * 4 + (lane >> 4)) ^ (lane & 15);
      // every x read of the k-step first, then the multiplies (the reads' latencies overlap
      // instead of each pair being waited for before its two multiplies)
      bf16x8 av[MTW];
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) av[mt] = *(const bf16x8*)(xb + mt * 16 * GKC + slot * 8);
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
          if constexpr (F16)
            acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h16x8, av[mt]),
                                                                __builtin_bit_cast(h16x8, bq[p][t]), acc[mt][t], 0, 0, 0);
          else
            acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mt], bq[p][t], acc[mt][t], 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, MTW, 0);        // the LDS reads
      __builtin_amdgcn_sched_group_barrier(0x008, MTW * NT, 0);   // then the multiplies
      // keep the reloads here: the scheduler would otherwise sink them to the end of the chunk
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < NT; ++t) bq[p][t] = wload<PK>(wp[t] + (cw * GPF + p) * KS);
      __builtin_amdgcn_sched_barrier(0);
    }
    store_x((c + 1) & 1, xr);
    // LDS-only barrier: __syncthreads() would also wait for every weight fragment in flight
    lds_barrier();
  };
  for (int c = 0; c < nchunks; c += 2) {
    step(c, bqa);
    if (c + 1 < nchunks) step(c + 1, bqb);
  }
  gemm_finish<MTW, NT, NG * NT * 16, GW * 64, ROWS, F16>(a, acc, xs, mh * MTW, ng * NT * 16);
}

template <int MT, int NT, int GW, int MS>
size_t gemm_lds() {
  const size_t xbuf = 2 * (size_t)MT * 16 * GKC * 2;                      // x double buffer
  const size_t lgt = (size_t)MT * 16 * (GW / MS * NT * 16 + 8) * 2 +      // the block's logits,
                     ((size_t)MT * 16 + 1) * (KMAX * 4 + 8);              // staged winners' keys, (max, sum)
  return xbuf > lgt ? xbuf : lgt;
}

template <int MT, int NT, int GW, bool PK, bool F16, int MS>
int launch_gemm(const GemmArgs& a0, hipStream_t st) {
  // cfh_head_ws_bytes sizes the candidate lists for blocks of at least 128 columns
  static_assert(GW / MS * NT * 16 >= 128, "a GEMM block must cover at least 128 shortlist columns");
  GemmArgs a = a0;
  const int cols = GW / MS * NT * 16;
  a.nsets = (a.n + cols - 1) / cols;
  const size_t lds = gemm_lds<MT, NT, GW, MS>();
  if (lds > 160 * 1024) return CFH_E_UNSUPPORTED;
  CFH_HIP(hipFuncSetAttribute((const void*)k_head_gemm<MT, NT, GW, PK, F16, MS>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  hipLaunchKernelGGL((k_head_gemm<MT, NT, GW, PK, F16, MS>), dim3(a.nsets), dim3(GW * 64), lds, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

template <int MT, int NT, int GW, int MS>
int gemm_nsets(int n) { return (n + GW / MS * NT * 16 - 1) / (GW / MS * NT * 16); }

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
  const h16* pred;     // marginal hidden rows of this depth: row m uses pred + group(m) * pred_ld
  h16* hsum;           // [M][d] = fp16(pred + fp16(sum + b))
  int ks, M, d;
  long long pred_ld;
  int rows_per_pred;   // rows sharing one pred row (0: every row uses row 0)
  int row0;            // row of this launch's first row in the whole call (for the grouping)
};

// Four columns a thread (d % 4 == 0): every partial read is one 16-byte load, all of a thread's
// loads issued before its sums.
__global__ void __launch_bounds__(256) k_path_out(PathOutArgs a) {
  const size_t total = (size_t)a.M * a.d, per_kc = total, nq = total / 4;
  for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < nq; q += (size_t)gridDim.x * blockDim.x) {
    const size_t i = q * 4;
    float4 s = *(const float4*)(a.P + i);
    for (int kc = 1; kc < a.ks; ++kc) {
      const float4 t = *(const float4*)(a.P + kc * per_kc + i);
      s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
    }
    const int m = (int)(i / a.d), c = (int)(i - (size_t)m * a.d);
    const int g = a.rows_per_pred > 0 ? (a.row0 + m) / a.rows_per_pred : 0;
    const h16* pr = a.pred + (size_t)g * a.pred_ld + c;
    const float v[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) a.hsum[i + t] = (h16)((float)pr[t] + r16(v[t] + (float)a.bias[c + t]));
  }
}

// Workgroups of a k_path_out launch over M rows of d: one float4 column group a thread, at most 1024.
unsigned path_out_blocks(int M, int d) {
  const long long q = (long long)M * d / 4;
  return (unsigned)std::max(1LL, std::min(1024LL, (q + 255) / 256));
}

// The path head's two MLP layers for up to PATH_CHUNK rows, each as one launch: one workgroup per
// 16-column tile whose WK waves each stream 1/WK of K (PF fragments in flight), the wave sums
// added in LDS, the epilogue applied in place of the separate partial-sum kernels:
//   PG_GELU    g = fp16(gelu(fp16(acc + b)))                         (mlp.0 -> GELU)
//   PG_PATHOUT hsum = fp16(pred[group(m)] + fp16(acc + b))             (mlp.3, then + the marginal hidden)
// The activation rows are read straight from global memory by each lane (every workgroup reads the
// same few rows, which stay in L2); lanes of rows past M re-read row M-1 and store nothing.
enum { PG_GELU = 0, PG_PATHOUT = 1 };

struct PathGemvArgs {
  const h16x8* w;      // packed [N][K]
  const h16* a;        // activation rows [M][K]
  const h16* bias;     // [N]
  h16* out;            // [M][N]
  const h16* pred;     // PG_PATHOUT: the marginal hidden rows (row g at pred + g * pred_ld)
  long long pred_ld;
  int rows_per_pred;   // rows sharing one pred row (0: every row uses row 0)
  int row0;            // the first row's index in the whole call (for the grouping)
  int M, N, K;
};

template <int EPI, int WK, int PFK>
__global__ void __launch_bounds__(WK * 64) k_path_gemv(PathGemvArgs g) {
  __shared__ f32x4 red[WK][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x;
  const int ksteps = g.K / 32, per = ksteps / WK, s0 = wave * per;
  const int row = lane & 15, kg = lane >> 4;
  const h16* arow = g.a + (size_t)min(row, g.M - 1) * g.K + (size_t)s0 * 32 + kg * 8;
  const h16x8* wp = g.w + ((size_t)t * ksteps + s0) * 64 + lane;
  h16x8 bw[PFK], ba[PFK];
#pragma unroll
  for (int p = 0; p < PFK; ++p) {
    bw[p] = __builtin_nontemporal_load(wp + (size_t)p * 64);
    ba[p] = *(const h16x8*)(arow + p * 32);
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int s = 0;
  for (; s < per - PFK; s += PFK) {
#pragma unroll
    for (int p = 0; p < PFK; ++p) {
      acc = mfma_f16(ba[p], bw[p], acc);
      bw[p] = __builtin_nontemporal_load(wp + (size_t)(s + PFK + p) * 64);
      ba[p] = *(const h16x8*)(arow + (s + PFK + p) * 32);
    }
  }
#pragma unroll
  for (int p = 0; p < PFK; ++p) acc = mfma_f16(ba[p], bw[p], acc);
  red[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  f32x4 v = red[0][lane];
#pragma unroll
  for (int w = 1; w < WK; ++w) {
    const f32x4 u = red[w][lane];
    v[0] += u[0]; v[1] += u[1]; v[2] += u[2]; v[3] += u[3];
  }
  const int n = t * 16 + (lane & 15), rbase = 4 * (lane >> 4);
  const float b = (float)g.bias[n];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = rbase + j;
    if (m >= g.M) continue;
    if constexpr (EPI == PG_GELU) {
      g.out[(size_t)m * g.N + n] = (h16)gelu_erf(r16(v[j] + b));
    } else {
      const int grp = g.rows_per_pred > 0 ? (g.row0 + m) / g.rows_per_pred : 0;
      g.out[(size_t)m * g.N + n] = (h16)((float)g.pred[(size_t)grp * g.pred_ld + n] + r16(v[j] + b));
    }
  }
}

// (WK, PF) of a path_gemv launch over `tiles` tiles and K: a whole number of PF-fragment blocks a
// wave, and as close to 2048 waves as the choices allow; 0 if none fits.
int path_gemv_shape(int tiles, int K, int* wk, int* pf) {
  static const int cand[][2] = {{8, 8}, {4, 8}, {8, 4}, {4, 4}, {2, 8}, {2, 4}};
  int best = -1;
  long long best_waves = 0;
  for (int i = 0; i < 6; ++i) {
    const int w = cand[i][0], f = cand[i][1], steps = K / 32;
    if (K % 32 || steps % w || (steps / w) % f || steps / w < f) continue;
    const long long waves = (long long)tiles * w;
    const bool better_fit = best < 0 || (best_waves < 2048 ? waves > best_waves : (waves >= 2048 && waves < best_waves));
    if (better_fit) {
      best = i;
      best_waves = waves;
    }
  }
  if (best < 0) return 0;
  *wk = cand[best][0];
  *pf = cand[best][1];
  return 1;
}

template <int EPI>
int launch_path_gemv(const PathGemvArgs& g, hipStream_t st) {
  int wk = 0, pf = 0;
  if (g.N % 16 || g.M < 1 || g.M > 16 || !path_gemv_shape(g.N / 16, g.K, &wk, &pf)) return CFH_E_UNSUPPORTED;
  const dim3 grid((unsigned)(g.N / 16));
#define CFH_PG(W, F) \
  if (wk == W && pf == F) { hipLaunchKernelGGL((k_path_gemv<EPI, W, F>), grid, dim3(W * 64), 0, st, g); CFH_LAUNCH_CHECK(); return CFH_OK; }
  CFH_PG(8, 8) CFH_PG(4, 8) CFH_PG(8, 4) CFH_PG(4, 4) CFH_PG(2, 8) CFH_PG(2, 4)
#undef CFH_PG
  return CFH_E_UNSUPPORTED;
}

struct PathPlan {
  int o_ks, up_ks, dn_ks;
  bool fused;          // the MLP layers as two path_gemv launches (else split-K GEMVs + reductions)
  size_t off_P, off_a, off_up, off_g, off_dn, total;
};

PathPlan path_plan(int M, int d, int ffn, int order) {
  PathPlan p;
  const int pf = ffn * d;
  p.o_ks = ksplit_for(order, d / 16, d, M);
  p.up_ks = ksplit_for(1, pf / 16, d, M);
  p.dn_ks = ksplit_for(1, d / 16, pf, M);
  int wk, pfk;
  p.fused = path_gemv_shape(pf / 16, d, &wk, &pfk) && path_gemv_shape(d / 16, pf, &wk, &pfk);
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

// The path residual of many rows (the beams of a batch) in groups of up to WMAXR rows: every weight
// of the path head streams once per group through the wide kernel (cfh_wide.h) instead of once
// per 16 rows.  offsets: one k_wide launch over the live offset projections (the embedding rows
// gathered by the ancestor ids), split-K partials; k_path_sum; up: k_wide with the GELU epilogue
// (fp16 rounding before the GELU, as torch's Linear then GELU modules); down: split-K partials;
// k_path_out.
struct PathWide {
  bool ok;
  int o_ks, dn_ks, up_wv;
  size_t off_P, off_a, off_g, off_dn, total;
};

PathWide path_wide_plan(int M, int d, int ffn, int order) {
  PathWide p = {};
  const int pf = ffn * d;
  constexpr int CUS = 256, WV = 4;
  auto ks_for = [&](int units, int N, int K) {
    int best = 0;
    for (int ks = 1; ks <= K / WCH; ++ks) {
      if (K % ks || (K / ks) % WCH) continue;
      best = ks;
      if ((long long)units * (N / 16 / (WT * WV)) * ks >= CUS) break;
    }
    return best;
  };
  p.o_ks = ks_for(order, d, d);
  p.dn_ks = ks_for(1, d, pf);
  p.up_wv = wide_wv(pf / 16, 1);
  auto wa = [&](int nex, int N, int K, int ks) {
    WArgs a = {};
    a.nex = nex; a.N = N; a.K = K; a.ks = ks;
    return a;
  };
  p.ok = order <= 4 && p.o_ks > 0 && p.dn_ks > 0 && p.up_wv > 0 && !wide_check(wa(order, d, d, p.o_ks), WV, M) &&
         !wide_check(wa(1, pf, d, 1), p.up_wv, M) && !wide_check(wa(1, d, pf, p.dn_ks), WV, M);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = cfh::align256(off + bytes);
    return o;
  };
  p.off_P = take((size_t)order * p.o_ks * M * d * 4);
  p.off_a = take((size_t)M * d * 2);
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

// The beam step in three phases around two workgroup barriers, run by one wave (lane = 0 .. 63):
// the lane's candidate and the old frontier state into LDS; the k rounds of the wave's best; the
// winners' outputs.
struct BeamSmem {
  int old_lastp[64 * 8];   // F <= 64 frontier slots x order <= 8
  int old_prev[64];
  int win_flat[64];
  float win_val[64];
};

__device__ __forceinline__ void beam_phase1(const BeamArgs& a, int b, int lane, BeamSmem& s, float& cv, int& ci) {
  const int ncand = a.F * a.TB;
  cv = -INFINITY;
  ci = INT_MAX;
  if (lane < ncand) {
    const int f = lane / a.TB, jj = lane - f * a.TB;
    cv = a.cum[b * a.keep + f] + a.vals[((size_t)b * a.F + f) * a.TB + jj];
    ci = lane;
  }
  for (int q = lane; q < a.F * a.order; q += 64) s.old_lastp[q] = a.lastp[(size_t)b * a.keep * a.order + q];
  if (a.tree && lane < a.F) s.old_prev[lane] = a.prev_ids[b * a.keep + lane];
}

__device__ __forceinline__ void beam_phase2(int k, int lane, BeamSmem& s, float cv, int ci) {
  for (int r = 0; r < k; ++r) {
    float bv = cv;
    int bi = ci;
    group_best<64>(bv, bi);
    if (ci == bi) { cv = -INFINITY; ci = INT_MAX; }
    if (lane == 0) { s.win_val[r] = bv; s.win_flat[r] = bi; }
  }
}

__device__ __forceinline__ void beam_phase3(const BeamArgs& a, int b, int lane, const BeamSmem& s, int k) {
  if (lane < k) {
    const int flat = s.win_flat[lane];
    const int src = flat / a.TB;
    const int loc = a.ids[((size_t)b * a.F + src) * a.TB + (flat - src * a.TB)];
    const int tok = loc < 0 ? -1 : (a.sl ? a.sl[loc] : loc);
    a.cum[b * a.keep + lane] = s.win_val[lane];
    int* lp = a.lastp + ((size_t)b * a.keep + lane) * a.order;
    lp[0] = tok;
    for (int q = 1; q < a.order; ++q) lp[q] = s.old_lastp[src * a.order + q - 1];
    if (a.tree) {
      a.toks[(size_t)b * a.ld_out + a.base + lane] = tok;
      a.bps[(size_t)b * a.ld_out + a.base + lane] = s.old_prev[src];
      a.prev_ids[b * a.keep + lane] = a.base + lane;
    } else {
      a.toks[b * a.keep + lane] = tok;
      a.bps[b * a.keep + lane] = src;
    }
  }
}

__global__ void __launch_bounds__(64) k_beam_step(BeamArgs a) {
  __shared__ BeamSmem s;
  const int b = blockIdx.x, lane = threadIdx.x;
  const int k = min(a.keep, a.F * a.TB);
  float cv;
  int ci;
  beam_phase1(a, b, lane, s, cv, ci);
  __syncthreads();
  beam_phase2(k, lane, s, cv, ci);
  __syncthreads();
  beam_phase3(a, b, lane, s, k);
}

// The merge of the head's candidate lists and the chain beam step in one launch: workgroup b holds
// chain b's F beam rows, a wave each (k_merge_wave's row merge, values to vals / ids / lse as there),
// then its first wave runs the beam step on those rows (every wave meets the barriers).
template <int S>
__global__ void __launch_bounds__(256) k_merge_beam(MergeArgs m, BeamArgs a) {
  extern __shared__ __align__(16) float mw[];
  __shared__ BeamSmem s;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, b = blockIdx.x;
  merge_row<S>(m, b * a.F + wave, mw + (size_t)wave * m.nsets * m.k * 2);
  __syncthreads();                                       // the chain's rows in vals / ids
  const int k = min(a.keep, a.F * a.TB);
  float cv = 0.f;
  int ci = 0;
  if (wave == 0) beam_phase1(a, b, lane, s, cv, ci);
  __syncthreads();
  if (wave == 0) beam_phase2(k, lane, s, cv, ci);
  __syncthreads();
  if (wave == 0) beam_phase3(a, b, lane, s, k);
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

int launch_head(const HeadArgs& ha0, hipStream_t st, bool packed = false) {
  HeadArgs ha = ha0;
  const size_t lds = head_lds(ha.M, ha.d, ha.r);
  if (lds > 150 * 1024) return CFH_E_UNSUPPORTED;
  const void* fn = packed ? (const void*)k_head<true> : (const void*)k_head<false>;
  CFH_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  const int ntiles = (ha.n + 15) / 16;
  const dim3 grid((ntiles + HW - 1) / HW, max(ha.groups, 1));
  if (packed) hipLaunchKernelGGL(k_head<true>, grid, dim3(HW * 64), lds, st, ha);
  else hipLaunchKernelGGL(k_head<false>, grid, dim3(HW * 64), lds, st, ha);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// out[i] (16-byte vectors) of the packed image of rows sl[0..n) of w [.][K]; i < ntiles * 16 * K / 8
__global__ void k_pack_rows(const uint4* __restrict__ w, const int* __restrict__ sl, int n, int K,
                            uint4* __restrict__ out) {
  const int ntiles = (n + 15) / 16;
  const size_t total = (size_t)ntiles * 16 * K / 8;
  const int ks = K / 32;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i & 63);
    const size_t ts = i >> 6;
    const int s = (int)(ts % ks);
    const int t = (int)(ts / ks);
    const int j = min(t * 16 + (lane & 15), n - 1);
    const size_t row = sl ? (size_t)sl[j] : (size_t)j;
    out[i] = w[(row * K + (size_t)s * 32 + 8 * (lane >> 4)) / 8];
  }
}

int launch_pack_rows(const void* w, const int32_t* sl, int n, int K, void* out, hipStream_t st) {
  const size_t total = (size_t)((n + 15) / 16) * 16 * K / 8;
  const int grid = (int)std::min<size_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(k_pack_rows, dim3(grid), dim3(256), 0, st, (const uint4*)w, sl, n, K, (uint4*)out);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

template <int S>
int launch_merge_wave(const MergeArgs& m, size_t row_bytes, hipStream_t st) {
  // one row (one wave) a workgroup, so the rows spread over the CUs (measured: 11.7 us for 160
  // rows against 13.4 us at four rows a workgroup)
  CFH_HIP(hipFuncSetAttribute((const void*)k_merge_wave<S>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)row_bytes));
  hipLaunchKernelGGL(k_merge_wave<S>, dim3(m.M), dim3(64), row_bytes, st, m);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int launch_merge(const void* ws, int M, int nsets, int k, float* vals, int* ids, float* lse, hipStream_t st) {
  MergeArgs m = {};
  m.ws = ws; m.M = M; m.nsets = nsets; m.k = k; m.vals = vals; m.ids = ids; m.lse = lse;
  const size_t row_bytes = (size_t)nsets * k * 8;
  if (row_bytes <= MW_LDS) {
    const int S = (nsets + 63) / 64;
    if (S <= 1) return launch_merge_wave<1>(m, row_bytes, st);
    if (S <= 2) return launch_merge_wave<2>(m, row_bytes, st);
    if (S <= 4) return launch_merge_wave<4>(m, row_bytes, st);
    if (S <= 8) return launch_merge_wave<8>(m, row_bytes, st);
  }
  hipLaunchKernelGGL(k_topk_merge, dim3(M), dim3(MT_THREADS), 0, st, m);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

template <bool PK, bool F16>
int gemm_topk(const void* x, int M, int d, const void* W, const int32_t* sl, int n, const void* bias, int k,
              void* logits, float* vals, int32_t* ids, float* lse, void* ws, hipStream_t st) {
  if (!x || !W || M < 1 || M > 256 || d < GKC || d % GKC || n < 1 || k < 0 || k > KMAX) return CFH_E_INVALID;
  if (k == 0 ? !logits : (!vals || !ids || !ws)) return CFH_E_INVALID;
  GemmArgs ga = {};
  ga.x = (const uint16_t*)x; ga.W = (const uint16_t*)W; ga.sl = sl; ga.logits = (uint16_t*)logits; ga.ws = ws;
  ga.bias = (const uint16_t*)bias;
  ga.M = M; ga.d = d; ga.n = n; ga.k = k;
  int rc, nsets;
  if (M <= 64) {
    nsets = gemm_nsets<4, 2, 8, 1>(n);
    ga.nsets = nsets;
    rc = launch_gemm<4, 2, 8, PK, F16, 1>(ga, st);
  } else if (M <= 160) {
    nsets = gemm_nsets<10, GEMM160_NT, 8, GEMM160_MS>(n);
    ga.nsets = nsets;
    rc = launch_gemm<10, GEMM160_NT, 8, PK, F16, GEMM160_MS>(ga, st);
  } else {
    nsets = gemm_nsets<16, 1, 8, 1>(n);
    ga.nsets = nsets;
    rc = launch_gemm<16, 1, 8, PK, F16, 1>(ga, st);
  }
  if (rc || k == 0) return rc;
  return launch_merge(ws, M, nsets, k, vals, ids, lse, st);
}

int head_args(HeadArgs& ha, const void* h, int M, int d, const void* W, const int32_t* sl, int n, const void* a,
              const int32_t* a_ids, int a_ids_stride, int r, const void* W2) {
  if (!h || !W || M < 1 || M > HMAXM || d < 32 || d % 256 || n < 1) return CFH_E_INVALID;
  if (W2 && (!a || r < 32 || r % 256)) return CFH_E_INVALID;
  ha = HeadArgs{};
  ha.h = (const h16*)h; ha.W = (const h16*)W; ha.sl = sl; ha.a = (const h16*)a; ha.a_ids = a_ids;
  ha.W2 = (const h16*)W2; ha.M = M; ha.d = d; ha.n = n; ha.r = W2 ? r : 0;
  ha.a_ids_stride = a_ids_stride > 0 ? a_ids_stride : 1;
  ha.groups = 1;
  return CFH_OK;
}

// Depth 0 of a search (one thread per (request, beam)): lastp = -1 but for the committed token in
// position 0 (every beam of a chain, beam 0 of a tree), cum = 0 for beam 0 and -inf for the others
// (chain) or 0 (tree), prev_ids = -1 (tree).
struct BeamInitArgs {
  const int64_t* known0;
  int32_t* lastp;
  float* cum;
  int32_t* prev_ids;
  int B, W, order, tree;
};

__global__ void __launch_bounds__(256) k_beam_init(BeamInitArgs a) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.B * a.W) return;
  const int b = i / a.W, w = i - b * a.W;
  int32_t* lp = a.lastp + (size_t)i * a.order;
  lp[0] = (!a.tree || w == 0) ? (int32_t)a.known0[b] : -1;
  for (int j = 1; j < a.order; ++j) lp[j] = -1;
  a.cum[i] = (a.tree || w == 0) ? 0.f : -INFINITY;
  if (a.tree) a.prev_ids[i] = -1;
}

}  // namespace

extern "C" {

int64_t cfh_head_ws_bytes(int M, int n, int k) {
  if (M < 1 || n < 1 || k < 1 || k > KMAX) return -1;
  const int nsets = (n + 127) / 128;    // the narrowest column block of any head kernel
  return (int64_t)cand_bytes(M, nsets, k);
}

int cfh_head_logits(const void* h, int M, int d, const void* W, const int32_t* sl, int n, const void* a,
                    const int32_t* a_ids, int a_ids_stride, int r, const void* W2, void* logits, void* stream) {
  if (!logits) return CFH_E_INVALID;
  HeadArgs ha;
  int rc = head_args(ha, h, M, d, W, sl, n, a, a_ids, a_ids_stride, r, W2);
  if (rc) return rc;
  ha.logits = (h16*)logits;
  return launch_head(ha, (hipStream_t)stream);
}

int cfh_row_topk(const void* logits, int M, int n, int k, float* vals, int32_t* ids, float* lse, void* stream) {
  if (!logits || !vals || !ids || M < 1 || n < 1 || k < 1 || k > KMAX) return CFH_E_INVALID;
  TopkArgs ta = {};
  ta.logits = (const h16*)logits; ta.ld = n; ta.M = M; ta.n = n; ta.k = k; ta.vals = vals; ta.ids = ids; ta.lse = lse;
  hipLaunchKernelGGL(k_topk, dim3(M), dim3(TK_THREADS), 0, (hipStream_t)stream, ta);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int cfh_head_topk(const void* h, int M, int d, const void* W, const int32_t* sl, int n, const void* a,
                  const int32_t* a_ids, int a_ids_stride, int r, const void* W2, int k, void* logits, float* vals,
                  int32_t* ids, float* lse, void* ws, void* stream) {
  if (!vals || !ids || !ws || k < 1 || k > KMAX) return CFH_E_INVALID;
  HeadArgs ha;
  int rc = head_args(ha, h, M, d, W, sl, n, a, a_ids, a_ids_stride, r, W2);
  if (rc) return rc;
  ha.logits = (h16*)logits;
  ha.ws = ws;
  ha.k = k;
  ha.nsets = (n + HCOLS - 1) / HCOLS;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = launch_head(ha, st))) return rc;
  return launch_merge(ws, M, ha.nsets, k, vals, ids, lse, st);
}

int64_t cfh_head_packed_bytes(int n, int d, int r) {
  if (n < 1 || d < 32 || d % 256 || r < 0 || (r > 0 && (r < 32 || r % 256))) return -1;
  return (int64_t)(head_packed_w_bytes(n, d) + (r > 0 ? head_packed_w_bytes(n, r) : 0));
}

int cfh_head_pack(const void* W, const void* W2, const int32_t* sl, int n, int d, int r, void* packed,
                  void* stream) {
  if (!W || !packed || cfh_head_packed_bytes(n, d, r) < 0 || (r > 0 && !W2)) return CFH_E_INVALID;
  hipStream_t st = (hipStream_t)stream;
  int rc = launch_pack_rows(W, sl, n, d, packed, st);
  if (rc || r == 0) return rc;
  return launch_pack_rows(W2, sl, n, r, (char*)packed + head_packed_w_bytes(n, d), st);
}

int cfh_head_topk_packed(const void* h, int M, int d, const void* packed, int n, const void* a,
                         const int32_t* a_ids, int a_ids_stride, int r, int k, void* logits, float* vals,
                         int32_t* ids, float* lse, void* ws, void* stream) {
  if (!packed || !vals || !ids || !ws || k < 1 || k > KMAX || cfh_head_packed_bytes(n, d, r) < 0) return CFH_E_INVALID;
  const void* W2 = r > 0 ? (const char*)packed + head_packed_w_bytes(n, d) : nullptr;
  HeadArgs ha;
  int rc = head_args(ha, h, M, d, packed, nullptr, n, a, a_ids, a_ids_stride, r, W2);
  if (rc) return rc;
  ha.logits = (h16*)logits;
  ha.ws = ws;
  ha.k = k;
  ha.nsets = (n + HCOLS - 1) / HCOLS;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = launch_head(ha, st, true))) return rc;
  return launch_merge(ws, M, ha.nsets, k, vals, ids, lse, st);
}

int cfh_head_topk_packed_beam_chain(const void* h, int M, int d, const void* packed, int n, const void* a,
                                    const int32_t* a_ids, int a_ids_stride, int r, float* vals, int32_t* ids,
                                    float* lse, void* ws, float* cum, int32_t* lastp, const int32_t* sl,
                                    int32_t* toks, int32_t* bps, int B, int W, int order, void* stream) {
  if (!packed || !vals || !ids || !ws || !cum || !lastp || !toks || !bps || B < 1 || W < 1 || W * W > 64 ||
      W > KMAX || order < 1 || order > 8 || M != B * W || cfh_head_packed_bytes(n, d, r) < 0)
    return CFH_E_INVALID;
  const void* W2 = r > 0 ? (const char*)packed + head_packed_w_bytes(n, d) : nullptr;
  HeadArgs ha;
  int rc = head_args(ha, h, M, d, packed, nullptr, n, a, a_ids, a_ids_stride, r, W2);
  if (rc) return rc;
  ha.logits = nullptr;
  ha.ws = ws;
  ha.k = W;
  ha.nsets = (n + HCOLS - 1) / HCOLS;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = launch_head(ha, st, true))) return rc;
  BeamArgs ba = {};
  ba.vals = vals; ba.ids = ids; ba.cum = cum; ba.lastp = lastp; ba.sl = sl; ba.toks = toks; ba.bps = bps;
  ba.B = B; ba.F = W; ba.TB = W; ba.keep = W; ba.order = order; ba.tree = 0;
  MergeArgs mg = {};
  mg.ws = ws; mg.M = M; mg.nsets = ha.nsets; mg.k = W; mg.vals = vals; mg.ids = ids; mg.lse = lse;
  const size_t row_bytes = (size_t)ha.nsets * W * 8;
  const int S = (ha.nsets + 63) / 64;
  if (W <= 4 && S <= 8 && row_bytes * W <= 150 * 1024) {
    const size_t lds = row_bytes * W;
#define CFH_MB(SS)                                                                                          \
  if (S <= SS) {                                                                                            \
    CFH_HIP(hipFuncSetAttribute((const void*)k_merge_beam<SS>, hipFuncAttributeMaxDynamicSharedMemorySize,  \
                                (int)lds));                                                                 \
    hipLaunchKernelGGL(k_merge_beam<SS>, dim3(B), dim3(W * 64), lds, st, mg, ba);                          \
    CFH_LAUNCH_CHECK();                                                                                     \
    return CFH_OK;                                                                                          \
  }
    CFH_MB(1) CFH_MB(2) CFH_MB(4) CFH_MB(8)
#undef CFH_MB
  }
  if ((rc = launch_merge(ws, M, ha.nsets, W, vals, ids, lse, st))) return rc;
  hipLaunchKernelGGL(k_beam_step, dim3(B), dim3(64), 0, st, ba);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int cfh_head_gemm_topk(const void* x, int M, int d, const void* W, const int32_t* sl, int n, int k, void* logits,
                       float* vals, int32_t* ids, float* lse, void* ws, void* stream) {
  if (k < 1) return CFH_E_INVALID;
  return gemm_topk<false, false>(x, M, d, W, sl, n, nullptr, k, logits, vals, ids, lse, ws, (hipStream_t)stream);
}

int cfh_head_gemm_topk_packed(const void* x, int M, int d, const void* packed, int n, int k, void* logits,
                              float* vals, int32_t* ids, float* lse, void* ws, void* stream) {
  if (cfh_head_packed_bytes(n, d, 0) < 0) return CFH_E_INVALID;
  if (k < 1) return CFH_E_INVALID;
  return gemm_topk<true, false>(x, M, d, packed, nullptr, n, nullptr, k, logits, vals, ids, lse, ws,
                                (hipStream_t)stream);
}

int cfh_head_topk_grouped(const void* h, int G, int M, int d, const void* W, const int32_t* sl, long long sl_stride,
                          int n, const void* a, const int32_t* a_ids, int a_ids_stride, int r, const void* W2, int k,
                          float* vals, int32_t* ids, float* lse, void* ws, void* stream) {
  if (!vals || !ids || !ws || !sl || G < 1 || G > 65535 || sl_stride < n || k < 1 || k > KMAX) return CFH_E_INVALID;
  HeadArgs ha;
  int rc = head_args(ha, h, M, d, W, sl, n, a, a_ids, a_ids_stride, r, W2);
  if (rc) return rc;
  ha.ws = ws;
  ha.k = k;
  ha.nsets = (n + HCOLS - 1) / HCOLS;
  ha.groups = G;
  ha.sl_stride = sl_stride;
  hipStream_t st = (hipStream_t)stream;
  if ((rc = launch_head(ha, st))) return rc;
  return launch_merge(ws, G * M, ha.nsets, k, vals, ids, lse, st);
}

int cfh_head_gemm16_topk(const void* x, int M, int d, const void* packed, int n, const void* bias, int k,
                         void* logits, float* vals, int32_t* ids, float* lse, void* ws, void* stream) {
  if (cfh_head_packed_bytes(n, d, 0) < 0) return CFH_E_INVALID;
  return gemm_topk<true, true>(x, M, d, packed, nullptr, n, bias, k, logits, vals, ids, lse, ws,
                               (hipStream_t)stream);
}

int64_t cfh_path_ws_bytes(int M, int d, int ffn_mult, int order) {
  if (M < 1 || d < 512 || d % 512 || ffn_mult < 1 || order < 1 || order > MAXEX) return -1;
  size_t total = path_plan(std::min(M, PATH_CHUNK), d, ffn_mult, order).total;
  if (M > PATH_CHUNK) {
    const PathWide pw = path_wide_plan(std::min(M, WMAXR), d, ffn_mult, order);
    if (pw.ok) total = std::max(total, pw.total);
  }
  return (int64_t)total;
}

// One launch sequence of the path residual for a wide group of M <= WMAXR rows.
static int path_group_wide(const PathWide& pw, const void* const* ph, int order, int ffn_mult, int d,
                           const int32_t* lastp, int M, int o, const void* embed_w, const void* pred, long long pred_ld,
                           int rows_per_pred, int row0, void* hsum, void* ws, hipStream_t st) {
  const int pf = ffn_mult * d;
  char* base = (char*)ws;
  float* P = (float*)(base + pw.off_P);
  h16* A = (h16*)(base + pw.off_a);
  h16* G = (h16*)(base + pw.off_g);
  float* Pdn = (float*)(base + pw.off_dn);
  int rc;
  if (o > 0) {
    WArgs a = {};
    a.nex = o; a.N = d; a.K = d; a.ks = pw.o_ks;
    for (int j = 0; j < o; ++j) {
      WEx& x = a.ex[j];
      x.w = (const h16x8*)ph[j]; x.a = (const h16*)embed_w; x.lda = d; x.ids = lastp + j; x.ids_stride = order;
      x.out = P + (size_t)j * pw.o_ks * M * d; x.S = M;
    }
    if ((rc = launch_wide<E_PART>(a, 4, st))) return rc;
  }
  PathSumArgs ps = {};
  ps.P = P; ps.lastp = lastp; ps.g = (const h16*)ph[2 * order]; ps.b = (const h16*)ph[2 * order + 1]; ps.a = A;
  ps.order = order; ps.o = o; ps.ks = pw.o_ks; ps.M = M; ps.d = d;
  for (int j = 0; j < o; ++j) ps.bias[j] = (const h16*)ph[order + j];
  hipLaunchKernelGGL(k_path_sum, dim3(M), dim3(ROWT), 0, st, ps);
  CFH_LAUNCH_CHECK();
  {
    WArgs a = {};
    a.nex = 1; a.N = pf; a.K = d; a.ks = 1; a.gelu_r16 = 1;
    a.ex[0].w = (const h16x8*)ph[2 * order + 2]; a.ex[0].a = A; a.ex[0].lda = d;
    a.ex[0].bias = (const h16*)ph[2 * order + 3]; a.ex[0].out = G; a.ex[0].S = M;
    if ((rc = launch_wide<E_GELU16>(a, pw.up_wv, st))) return rc;
  }
  {
    WArgs a = {};
    a.nex = 1; a.N = d; a.K = pf; a.ks = pw.dn_ks;
    a.ex[0].w = (const h16x8*)ph[2 * order + 4]; a.ex[0].a = G; a.ex[0].lda = pf; a.ex[0].out = Pdn; a.ex[0].S = M;
    if ((rc = launch_wide<E_PART>(a, 4, st))) return rc;
  }
  PathOutArgs po = {};
  po.P = Pdn; po.bias = (const h16*)ph[2 * order + 5]; po.pred = (const h16*)pred; po.hsum = (h16*)hsum;
  po.ks = pw.dn_ks; po.M = M; po.d = d; po.pred_ld = pred_ld; po.rows_per_pred = rows_per_pred; po.row0 = row0;
  hipLaunchKernelGGL(k_path_out, dim3(path_out_blocks(M, d)), dim3(256), 0, st, po);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// One launch sequence of the path residual for M <= PATH_CHUNK rows (rows row0 .. of the call).
static int path_chunk(const PathPlan& pp, const void* const* ph, int order, int ffn_mult, int d, const int32_t* lastp, int M,
               int o, const void* embed_w, const void* pred, long long pred_ld, int rows_per_pred, int row0,
               void* hsum, void* ws, hipStream_t st) {
  const int pf = ffn_mult * d;
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
  if (pp.fused) {
    PathGemvArgs g = {};
    g.w = W0; g.a = A; g.bias = b0; g.out = G; g.M = M; g.N = pf; g.K = d;
    if ((rc = launch_path_gemv<PG_GELU>(g, st))) return rc;
    g.w = W3; g.a = G; g.bias = b3; g.out = (h16*)hsum; g.N = d; g.K = pf;
    g.pred = (const h16*)pred; g.pred_ld = pred_ld; g.rows_per_pred = rows_per_pred; g.row0 = row0;
    return launch_path_gemv<PG_PATHOUT>(g, st);
  }
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
  po.pred_ld = pred_ld; po.rows_per_pred = rows_per_pred; po.row0 = row0;
  hipLaunchKernelGGL(k_path_out, dim3(path_out_blocks(M, d)), dim3(256), 0, st, po);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int cfh_path_residual(const void* const* ph, int order, int ffn_mult, int d, const int32_t* lastp, int M,
                      int nlive, const void* embed_w, const void* pred, long long pred_ld, int rows_per_pred,
                      void* hsum, void* ws, void* stream) {
  if (!ph || !lastp || !embed_w || !pred || !hsum || !ws) return CFH_E_INVALID;
  if (M < 1 || d < 512 || d % 512 || ffn_mult < 1 || order < 1 || order > MAXEX) return CFH_E_INVALID;
  if (rows_per_pred < 0 || pred_ld < 0) return CFH_E_INVALID;
  const int n_ptr = 2 * order + 6;
  for (int i = 0; i < n_ptr; ++i)
    if (!ph[i]) return CFH_E_INVALID;
  const int o = (nlive < 0 || nlive > order) ? order : nlive;
  if (M > PATH_CHUNK) {
    // many rows (a batch's beams): wide groups of up to WMAXR rows, balanced
    const PathWide pw = path_wide_plan(std::min(M, WMAXR), d, ffn_mult, order);
    if (pw.ok) {
      const int ng = (M + WMAXR - 1) / WMAXR, per = (M + ng - 1) / ng;
      for (int r0 = 0; r0 < M; r0 += per) {
        const int m = std::min(per, M - r0);
        const int rc = path_group_wide(pw, ph, order, ffn_mult, d, lastp + (size_t)r0 * order, m, o, embed_w, pred,
                                       pred_ld, rows_per_pred, r0, (h16*)hsum + (size_t)r0 * d, ws,
                                       (hipStream_t)stream);
        if (rc) return rc;
      }
      return CFH_OK;
    }
  }
  const PathPlan pp = path_plan(std::min(M, PATH_CHUNK), d, ffn_mult, order);
  // the GEMVs take at most PATH_CHUNK activation rows: chunks run one after another on the stream,
  // each on the same workspace
  for (int r0 = 0; r0 < M; r0 += PATH_CHUNK) {
    const int m = std::min(PATH_CHUNK, M - r0);
    const int rc = path_chunk(pp, ph, order, ffn_mult, d, lastp + (size_t)r0 * order, m, o, embed_w, pred, pred_ld,
                              rows_per_pred, r0, (h16*)hsum + (size_t)r0 * d, ws, (hipStream_t)stream);
    if (rc) return rc;
  }
  return CFH_OK;
}

int cfh_beam_init(const int64_t* known0, int32_t* lastp, float* cum, int32_t* prev_ids, int B, int W, int order,
                  int tree, void* stream) {
  if (!known0 || !lastp || !cum || (tree && !prev_ids) || B < 1 || W < 1 || W > 64 || order < 1 || order > 8)
    return CFH_E_INVALID;
  BeamInitArgs a = {};
  a.known0 = known0; a.lastp = lastp; a.cum = cum; a.prev_ids = prev_ids; a.B = B; a.W = W; a.order = order;
  a.tree = tree;
  hipLaunchKernelGGL(k_beam_init, dim3((B * W + 255) / 256), dim3(256), 0, (hipStream_t)stream, a);
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
