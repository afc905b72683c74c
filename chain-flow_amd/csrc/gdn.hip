// Tree-aware gated delta net (GDN) state update for tree verification on MI355X.
//
// Reference semantics (cf/ = src/chain_flow/): cf/kernels/tree_scan.py:23-73 -- every node n of a
// BFS-ordered draft tree (parent[n] < n, -1 = root) starts from its parent's state (roots from S0):
//     S = S_parent * exp(g);  delta = (v - S^T k) * beta;  S = S + k (x) delta;  o = S^T q
// with q, k l2-normalised (x / (|x| + 1e-6), or x / sqrt(|x|^2 + 1e-6) as in the Triton kernels of
// cf/vllm_tree/tree_ssm.py:60-62) and q scaled by Dk^-1/2.  State layout [H][Dk][Dv].
//
// Execution plan (path-parallel): one workgroup per (node, head, 64-column value slice), four
// waves of it each holding 32 of the Dk = 128 state rows (lane j: column j) in registers.  The
// workgroup replays the node's ancestor chain from the root, so every node's state and output come
// from the same sequential per-path recurrence (tree_scan.py:78-90) and no workgroup waits for
// another; each step's dot products are summed over the four waves through LDS.  k of each path
// step is normalised once and broadcast through LDS; q only for the node itself (the output).
// The recompute costs depth x 3 Dk FMA-class operations per column per node, below the state
// traffic (S0 read, node state written).
#include "cfh_common.h"
#include "cfh_host.h"

namespace {

constexpr int GDN_DK = 128;
constexpr int GDN_MAXN = 256;

struct GdnArgs {
  const uint16_t* q;     // [N][H][Dk] bf16
  const uint16_t* k;     // [N][H][Dk] bf16
  const uint16_t* v;     // [N][H][Dv] bf16
  const float* g;        // [N][H] log decay
  const float* beta;     // [N][H]
  const float* S0;       // [H][Dk][Dv]
  const int* parent;     // [N]
  float* out;            // [N][H][Dv]
  float* states;         // [N][H][Dk][Dv] or null
  int N, H, Dv, l2norm, l2mode;
  float scale;
};

__device__ __forceinline__ float bf16f(uint16_t b) { return __uint_as_float((unsigned)b << 16); }

// The ancestor chain comes from the parents staged in LDS by one coalesced load; each batch of up to
// GDN_LB path steps issues all its loads (k, v, gates) before any math, and the step scalars wait
// in LDS for the sequential replay.  The dot products over Dk run as four partial sums.
constexpr int GDN_LB = 8;

// Lane 0 walks n, parent(n), ..., root through the staged parents; *len = path length, returns
// nonzero if a parent does not precede its child (not BFS-ordered).
__device__ int gdn_path(const int* __restrict__ parent, int n, int* par, int* path, int* plen_s, int* bad_s) {
  for (int i = threadIdx.x; i <= n; i += blockDim.x) par[i] = parent[i];
  __syncthreads();
  if (threadIdx.x == 0) {
    int len = 0, bad = 0, cur = n;
    while (true) {
      path[len++] = cur;
      const int p = par[cur];
      if (p < 0) break;
      if (p >= cur) { bad = 1; break; }
      cur = p;
    }
    *plen_s = len;
    *bad_s = bad;
  }
  __syncthreads();
  return *bad_s;
}

// GDN_NW waves per (node, head, 64-column value slice): wave w holds state rows
// [GDN_HK w, GDN_HK (w + 1)) of the slice's columns, so the deepest nodes' replays (the critical
// path) spread over GDN_NW times the SIMDs.  Each step's dot product is the sum of the waves'
// partials, exchanged through LDS (one barrier a step, buffers alternating by step).
constexpr int GDN_NW = 4;                  // waves per (node, head, value slice)
constexpr int GDN_HK = GDN_DK / GDN_NW;    // state rows a wave holds

// kv partial = S^T k over the wave's rows after S *= e (k broadcast from LDS), four partial sums
__device__ __forceinline__ float gdn_decay_dot_h(float* S, const float* kk, float e) {
  float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
  for (int i = 0; i < GDN_HK; i += 4) {
    const float4 k4 = *(const float4*)(kk + i);
    S[i] *= e; S[i + 1] *= e; S[i + 2] *= e; S[i + 3] *= e;
    p0 += S[i] * k4.x; p1 += S[i + 1] * k4.y; p2 += S[i + 2] * k4.z; p3 += S[i + 3] * k4.w;
  }
  return (p0 + p1) + (p2 + p3);
}

__device__ __forceinline__ float gdn_dot_h(const float* S, const float* qq) {
  float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
  for (int i = 0; i < GDN_HK; i += 4) {
    const float4 q4 = *(const float4*)(qq + i);
    p0 += S[i] * q4.x; p1 += S[i + 1] * q4.y; p2 += S[i + 2] * q4.z; p3 += S[i + 3] * q4.w;
  }
  return (p0 + p1) + (p2 + p3);
}

__device__ __forceinline__ void gdn_rank1_h(float* S, const float* kk, float delta) {
#pragma unroll
  for (int i = 0; i < GDN_HK; i += 4) {
    const float4 k4 = *(const float4*)(kk + i);
    S[i] += k4.x * delta; S[i + 1] += k4.y * delta; S[i + 2] += k4.z * delta; S[i + 3] += k4.w * delta;
  }
}

__global__ void __launch_bounds__(64 * GDN_NW) k_gdn_tree(GdnArgs a) {
  __shared__ __align__(16) float qs[GDN_DK];
  __shared__ __align__(16) float ks[GDN_LB][GDN_DK];
  __shared__ float egs[GDN_LB], bts[GDN_LB], vjs[GDN_LB][64];
  __shared__ float red[2][GDN_NW][64];                       // [step parity][wave][lane]
  __shared__ int par[GDN_MAXN], path[GDN_MAXN];
  __shared__ int plen_s, bad_s;
  const int nvs = a.Dv / 64;
  int u = blockIdx.x;
  const int vs = u % nvs;
  u /= nvs;
  const int h = u % a.H;
  const int n = u / a.H;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int j = vs * 64 + lane;
  const int i0 = wave * GDN_HK;                              // this wave's state rows

  // the node's own q (for the output) and the initial state do not depend on the path: issued
  // before the parents, they share its memory round trip
  const size_t qn = ((size_t)n * a.H + h) * GDN_DK;
  float q0 = bf16f(a.q[qn + lane]), q1 = bf16f(a.q[qn + 64 + lane]);
  float S[GDN_HK];
  const float* s0 = a.S0 + ((size_t)h * GDN_DK + i0) * a.Dv + j;
#pragma unroll
  for (int i = 0; i < GDN_HK; ++i) S[i] = s0[(size_t)i * a.Dv];
  if (gdn_path(a.parent, n, par, path, &plen_s, &bad_s)) {   // not BFS-ordered: NaN outputs
    const float nan = __builtin_nanf("");
    if (wave == 0) a.out[((size_t)n * a.H + h) * a.Dv + j] = nan;
    if (a.states)
      for (int i = 0; i < GDN_HK; ++i)
        a.states[(((size_t)n * a.H + h) * GDN_DK + i0 + i) * a.Dv + j] = nan;
    return;
  }
  const int len = plen_s;
  int rb = 0;                                                // red buffer of the next exchange

  for (int t0 = len - 1; t0 >= 0; t0 -= GDN_LB) {
    const int nb = min(GDN_LB, t0 + 1);                      // steps t0, t0 - 1, ..., t0 - nb + 1
    if (wave == 0) {                                         // wave 0 stages the batch for both
      float k0[GDN_LB], k1[GDN_LB], vj[GDN_LB], gg[GDN_LB], bb[GDN_LB];
#pragma unroll
      for (int b = 0; b < GDN_LB; ++b) {
        const int m = path[t0 - min(b, nb - 1)];             // past nb: a repeat, never used
        const size_t qk = ((size_t)m * a.H + h) * GDN_DK;
        k0[b] = bf16f(a.k[qk + lane]);
        k1[b] = bf16f(a.k[qk + 64 + lane]);
        vj[b] = bf16f(a.v[((size_t)m * a.H + h) * a.Dv + j]);
        gg[b] = a.g[(size_t)m * a.H + h];
        bb[b] = a.beta[(size_t)m * a.H + h];
      }
#pragma unroll
      for (int b = 0; b < GDN_LB; ++b) {
        if (b < nb) {
          float ik = 1.0f;
          if (a.l2norm) {
            const float sk = wave_sum(k0[b] * k0[b] + k1[b] * k1[b]);
            ik = a.l2mode ? 1.0f / sqrtf(sk + 1e-6f) : 1.0f / (sqrtf(sk) + 1e-6f);
          }
          ks[b][lane] = k0[b] * ik;
          ks[b][lane + 64] = k1[b] * ik;
          vjs[b][lane] = vj[b];
          if (lane == 0) { egs[b] = expf(gg[b]); bts[b] = bb[b]; }
        }
      }
    }
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
      red[rb][wave][lane] = gdn_decay_dot_h(S, ks[b] + i0, egs[b]);
      __syncthreads();
      float kv = 0.f;
#pragma unroll
      for (int w = 0; w < GDN_NW; ++w) kv += red[rb][w][lane];
      rb ^= 1;
      gdn_rank1_h(S, ks[b] + i0, (vjs[b][lane] - kv) * bts[b]);
    }
    __syncthreads();   // the batch's reads of ks / vjs are done before the next batch writes them
  }
  if (wave == 0) {
    if (a.l2norm) {
      const float sq = wave_sum(q0 * q0 + q1 * q1);
      const float iq = a.l2mode ? 1.0f / sqrtf(sq + 1e-6f) : 1.0f / (sqrtf(sq) + 1e-6f);
      q0 *= iq; q1 *= iq;
    }
    qs[lane] = q0 * a.scale;
    qs[lane + 64] = q1 * a.scale;
  }
  __syncthreads();
  red[rb][wave][lane] = gdn_dot_h(S, qs + i0);
  __syncthreads();
  if (wave == 0) {
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < GDN_NW; ++w) o += red[rb][w][lane];
    a.out[((size_t)n * a.H + h) * a.Dv + j] = o;
  }
  if (a.states) {
    float* st = a.states + (((size_t)n * a.H + h) * GDN_DK + i0) * a.Dv + j;
#pragma unroll
    for (int i = 0; i < GDN_HK; ++i) st[(size_t)i * a.Dv] = S[i];
  }
}

// ---------------------------------------------------------------------------- vLLM layout
// The serving form (cf/vllm_tree/tree_ssm.py:256-311, path-parallel; bit-identical by construction to
// the per-node slot form :34-77): q, k, v are rows of the post-conv `mixed_qkv` [N][2 H K + HV V]
// (q heads, k heads, then HV value heads; value head hv uses q/k head hv / (HV / H)); the gates come
// from the projections a, b [N][HV]:
//     g = -exp(A_log) * softplus(a + dt_bias)   (softplus(x) = x above 20)
//     beta = bf16(sigmoid(b))
// q, k are normalised as x / sqrt(|x|^2 + 1e-6) and q scaled by `scale`.  States live in slots of
// `ssm_state` [slots][HV][V][K] (value-major, bf16 or fp32).  Every node starts from the prefix slot
// and replays its root->node path; each ancestor's state is rounded to the storage type (exactly
// what storing and re-reading its slot does), the node's own state stays fp32 for its output and
// is stored to node_slots[n].  Output o [N][HV][V] bf16.
struct GdnVArgs {
  const uint16_t* qkv;   // [N][ld] bf16
  const uint16_t* ga;    // [N][HV] bf16
  const uint16_t* gb;    // [N][HV] bf16
  const float* A_log;    // [HV]
  const float* dt_bias;  // [HV]
  void* state;           // [slots][HV][V][K]
  const int* slots;      // [N]
  const int* parent;     // [N]
  uint16_t* out;         // [N][HV][V] bf16
  int* status;           // [1] or null: set to 1 when a node's slot is refused
  int N, H, HV, V, ld, prefix, nslots, bf16_state, l2norm;
  float scale;
};

// round to nearest even, as torch's cast does: gfx950 converts in hardware (v_cvt_pk_bf16_f32, two
// values an instruction), inf unchanged, NaN stays NaN
__device__ __forceinline__ float round_bf16(float x) { return (float)(__bf16)x; }
__device__ __forceinline__ uint16_t to_bf16(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }

// The serving form's state rows (one value row of K = 128 contiguous elements per lane; wave w
// holds K elements [GDN_HK w, GDN_HK (w + 1))) pass through LDS so that global memory sees the workgroup's
// 64 rows as one contiguous block of 16-byte chunks; rows are padded by 16 bytes in LDS (row stride
// RB + 16), which keeps the lanes' row reads on different banks.
template <typename T>
__device__ __forceinline__ void rows_in(const T* __restrict__ src, float* S, unsigned char* lds) {
  constexpr int RB = GDN_DK * (int)sizeof(T), RS = RB + 16, NC = 64 * RB / 16;   // 1024 or 2048 chunks
  const int t = threadIdx.x;
  constexpr int NT = 64 * GDN_NW, NB = NC / NT < 8 ? NC / NT : 8;   // threads; chunks a batch
  static_assert(NC % (NT * NB) == 0, "the block splits into whole batches");
#pragma unroll
  for (int c0 = 0; c0 < NC; c0 += NT * NB) {
    uint4 v[NB];
#pragma unroll
    for (int q = 0; q < NB; ++q) v[q] = ((const uint4*)src)[c0 + t + NT * q];
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int e = (c0 + t + NT * q) * 16;
      *(uint4*)(lds + (e / RB) * RS + e % RB) = v[q];
    }
  }
  __syncthreads();
  const unsigned char* row = lds + (t & 63) * RS + (t >> 6) * (RB / GDN_NW);
#pragma unroll
  for (int q = 0; q < RB / (16 * GDN_NW); ++q) {
    const uint4 u = *(const uint4*)(row + 16 * q);
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int e = 0; e < 8; ++e) S[8 * q + e] = __uint_as_float((w[e >> 1] >> (16 * (e & 1))) << 16);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) S[4 * q + e] = __uint_as_float(w[e]);
    }
  }
  __syncthreads();   // the rows are read before the buffer is reused
}

template <typename T>
__device__ __forceinline__ void rows_out(T* __restrict__ dst, const float* S, unsigned char* lds) {
  constexpr int RB = GDN_DK * (int)sizeof(T), RS = RB + 16, NC = 64 * RB / 16;
  const int t = threadIdx.x;
  unsigned char* row = lds + (t & 63) * RS + (t >> 6) * (RB / GDN_NW);
#pragma unroll
  for (int q = 0; q < RB / (16 * GDN_NW); ++q) {
    uint4 u;
    if constexpr (sizeof(T) == 2) {
      unsigned w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = (unsigned)to_bf16(S[8 * q + 2 * e]) | ((unsigned)to_bf16(S[8 * q + 2 * e + 1]) << 16);
      u = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      u = make_uint4(__float_as_uint(S[4 * q]), __float_as_uint(S[4 * q + 1]), __float_as_uint(S[4 * q + 2]),
                     __float_as_uint(S[4 * q + 3]));
    }
    *(uint4*)(row + 16 * q) = u;
  }
  __syncthreads();
#pragma unroll
  for (int c0 = 0; c0 < NC; c0 += 64 * GDN_NW) {
    const int c = c0 + t, e = c * 16;
    ((uint4*)dst)[c] = *(const uint4*)(lds + (e / RB) * RS + e % RB);
  }
}

__global__ void __launch_bounds__(64 * GDN_NW) k_gdn_tree_vllm(GdnVArgs a) {
  __shared__ __align__(16) float qs[GDN_DK];
  __shared__ float red[2][GDN_NW][64];                       // [step parity][wave][lane]
  __shared__ int par[GDN_MAXN], path[GDN_MAXN];
  __shared__ int plen_s, bad_s;
  // the state rows (before the replay and after it) share their buffer with the replay's staging
  struct Stage {
    float ks[GDN_LB][GDN_DK];
    float egs[GDN_LB], bts[GDN_LB], vjs[GDN_LB][64];
  };
  constexpr int ROWS_BYTES = 64 * (GDN_DK * 4 + 16);
  static_assert(sizeof(Stage) <= ROWS_BYTES, "staging fits in the row buffer");
  __shared__ __align__(16) unsigned char rows[ROWS_BYTES];
  Stage& sg = *(Stage*)rows;
  float (*ks)[GDN_DK] = sg.ks;
  float* egs = sg.egs;
  float* bts = sg.bts;
  float (*vjs)[64] = sg.vjs;
  const int nvs = a.V / 64;
  int u = blockIdx.x;
  const int vs = u % nvs;
  u /= nvs;
  const int hv = u % a.HV;
  const int n = u / a.HV;
  const int h = hv / (a.HV / a.H);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int j = vs * 64 + lane;
  const int i0 = wave * GDN_HK;                              // this wave's K elements
  const size_t srow = (size_t)a.HV * a.V * GDN_DK;                 // elements per slot
  const size_t sblk = ((size_t)hv * a.V + vs * 64) * GDN_DK;       // the workgroup's 64 rows in a slot

  // the node's own q (for the output) and the prefix state do not depend on the path: issued
  // before the parents, they share its memory round trip
  const uint16_t* rown = a.qkv + (size_t)n * a.ld;
  float q0 = bf16f(rown[(size_t)h * GDN_DK + lane]), q1 = bf16f(rown[(size_t)h * GDN_DK + 64 + lane]);
  float S[GDN_HK];
  if (a.bf16_state)
    rows_in((const uint16_t*)a.state + (size_t)a.prefix * srow + sblk, S, rows);
  else
    rows_in((const float*)a.state + (size_t)a.prefix * srow + sblk, S, rows);
  const float Aexp = expf(a.A_log[hv]), dtb = a.dt_bias[hv];
  // the node's slot must lie in ssm_state, differ from the prefix slot and from every other node's
  // (checked here rather than on the host, so that a caller never synchronises to validate them)
  const int my = a.slots[n];
  int clash = 0;
  for (int m = threadIdx.x; m < a.N; m += blockDim.x) clash |= m != n && a.slots[m] == my;
  clash = __syncthreads_or(clash);
  const bool refused = clash || my < 0 || my >= a.nslots || my == a.prefix;
  if (refused && a.status && threadIdx.x == 0) a.status[0] = 1;
  if (refused || gdn_path(a.parent, n, par, path, &plen_s, &bad_s)) {
    // refused slot or not BFS-ordered: NaN outputs, no slot written
    if (wave == 0) a.out[((size_t)n * a.HV + hv) * a.V + j] = 0x7fc0;
    return;
  }
  const int len = plen_s;
  int rb = 0;                                                // red buffer of the next exchange
  const size_t koff = (size_t)a.H * GDN_DK + (size_t)h * GDN_DK;
  const size_t voff = 2 * (size_t)a.H * GDN_DK + (size_t)hv * a.V + j;
  for (int t0 = len - 1; t0 >= 0; t0 -= GDN_LB) {
    const int nb = min(GDN_LB, t0 + 1);                      // steps t0, t0 - 1, ..., t0 - nb + 1
    if (wave == 0) {                                         // wave 0 stages the batch for both
      float k0[GDN_LB], k1[GDN_LB], vj[GDN_LB], xa[GDN_LB], xb[GDN_LB];
#pragma unroll
      for (int b = 0; b < GDN_LB; ++b) {
        const int m = path[t0 - min(b, nb - 1)];             // past nb: a repeat, never used
        const uint16_t* row = a.qkv + (size_t)m * a.ld;
        k0[b] = bf16f(row[koff + lane]);
        k1[b] = bf16f(row[koff + 64 + lane]);
        vj[b] = bf16f(row[voff]);
        xa[b] = bf16f(a.ga[(size_t)m * a.HV + hv]);
        xb[b] = bf16f(a.gb[(size_t)m * a.HV + hv]);
      }
#pragma unroll
      for (int b = 0; b < GDN_LB; ++b) {
        if (b < nb) {
          float ik = 1.0f;
          if (a.l2norm) ik = 1.0f / sqrtf(wave_sum(k0[b] * k0[b] + k1[b] * k1[b]) + 1e-6f);
          ks[b][lane] = k0[b] * ik;
          ks[b][lane + 64] = k1[b] * ik;
          vjs[b][lane] = vj[b];
          if (lane == 0) {
            const float x = xa[b] + dtb;
            const float sp = x <= 20.0f ? logf(1.0f + expf(x)) : x;
            egs[b] = expf(-Aexp * sp);
            bts[b] = round_bf16(1.0f / (1.0f + expf(-xb[b])));
          }
        }
      }
    }
    __syncthreads();
    for (int b = 0; b < nb; ++b) {
      red[rb][wave][lane] = gdn_decay_dot_h(S, ks[b] + i0, egs[b]);
      __syncthreads();
      float kv = 0.f;
#pragma unroll
      for (int w = 0; w < GDN_NW; ++w) kv += red[rb][w][lane];
      rb ^= 1;
      gdn_rank1_h(S, ks[b] + i0, (vjs[b][lane] - kv) * bts[b]);
      if (t0 - b > 0 && a.bf16_state) {   // an ancestor: its stored (bf16) state is what the child reads
#pragma unroll
        for (int i = 0; i < GDN_HK; ++i) S[i] = round_bf16(S[i]);
      }
    }
    __syncthreads();   // the batch's reads of ks / vjs are done before the next batch writes them
  }
  // output with the node's own q
  if (wave == 0) {
    if (a.l2norm) {
      const float iq = 1.0f / sqrtf(wave_sum(q0 * q0 + q1 * q1) + 1e-6f);
      q0 *= iq; q1 *= iq;
    }
    qs[lane] = q0 * a.scale;
    qs[lane + 64] = q1 * a.scale;
  }
  __syncthreads();
  red[rb][wave][lane] = gdn_dot_h(S, qs + i0);
  __syncthreads();
  if (wave == 0) {
    float o = 0.f;
#pragma unroll
    for (int w = 0; w < GDN_NW; ++w) o += red[rb][w][lane];
    a.out[((size_t)n * a.HV + hv) * a.V + j] = to_bf16(o);
  }
  const size_t dst = (size_t)a.slots[n] * srow + sblk;
  if (a.bf16_state)
    rows_out((uint16_t*)a.state + dst, S, rows);
  else
    rows_out((float*)a.state + dst, S, rows);
}

}  // namespace

extern "C" {

int cfh_gdn_tree(const void* q, const void* k, const void* v, const float* g, const float* beta, const float* S0,
                 const int32_t* parent, int N, int H, int Dk, int Dv, int use_l2norm, int l2mode, float* out,
                 float* states, void* stream) {
  if (!q || !k || !v || !g || !beta || !S0 || !parent || !out) return CFH_E_INVALID;
  if (N < 1 || N > GDN_MAXN || H < 1 || Dv < 64 || Dv % 64) return CFH_E_INVALID;
  if (Dk != GDN_DK) return CFH_E_UNSUPPORTED;
  GdnArgs a = {};
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v; a.g = g; a.beta = beta;
  a.S0 = S0; a.parent = parent; a.out = out; a.states = states; a.N = N; a.H = H; a.Dv = Dv;
  a.l2norm = use_l2norm ? 1 : 0; a.l2mode = l2mode ? 1 : 0; a.scale = 1.0f / sqrtf((float)Dk);
  const long long blocks = (long long)N * H * (Dv / 64);
  hipLaunchKernelGGL(k_gdn_tree, dim3((unsigned)blocks), dim3(64 * GDN_NW), 0, (hipStream_t)stream, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int cfh_gdn_tree_vllm(const void* mixed_qkv, const void* a, const void* b, const float* A_log, const float* dt_bias,
                      void* ssm_state, int state_bf16, int nslots, const int32_t* node_slots, const int32_t* parent,
                      int prefix_slot, int N, int H, int HV, int K, int V, int use_l2norm, float scale,
                      void* out, int32_t* status, void* stream) {
  if (!mixed_qkv || !a || !b || !A_log || !dt_bias || !ssm_state || !node_slots || !parent || !out)
    return CFH_E_INVALID;
  if (N < 1 || N > GDN_MAXN || H < 1 || HV < H || HV % H || V < 64 || V % 64 || prefix_slot < 0 ||
      prefix_slot >= nslots)
    return CFH_E_INVALID;
  if (K != GDN_DK) return CFH_E_UNSUPPORTED;
  GdnVArgs g = {};
  g.qkv = (const uint16_t*)mixed_qkv; g.ga = (const uint16_t*)a; g.gb = (const uint16_t*)b;
  g.A_log = A_log; g.dt_bias = dt_bias; g.state = ssm_state; g.slots = node_slots; g.parent = parent;
  g.out = (uint16_t*)out; g.N = N; g.H = H; g.HV = HV; g.V = V; g.ld = 2 * H * K + HV * V;
  g.prefix = prefix_slot; g.nslots = nslots; g.status = status; g.bf16_state = state_bf16 ? 1 : 0; g.l2norm = use_l2norm ? 1 : 0; g.scale = scale;
  const long long blocks = (long long)N * HV * (V / 64);
  hipLaunchKernelGGL(k_gdn_tree_vllm, dim3((unsigned)blocks), dim3(64 * GDN_NW), 0, (hipStream_t)stream, g);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

}  // extern "C"
