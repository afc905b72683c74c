// Tree-aware gated delta net (GDN) state update for tree verification on MI355X.
//
// Reference semantics (cf/ = src/chain_flow/): cf/kernels/tree_scan.py:23-73 -- every node n of a
// BFS-ordered draft tree (parent[n] < n, -1 = root) starts from its parent's state (roots from S0):
//     S = S_parent * exp(g);  delta = (v - S^T k) * beta;  S = S + k (x) delta;  o = S^T q
// with q, k l2-normalised (x / (|x| + 1e-6), or x / sqrt(|x|^2 + 1e-6) as in the Triton kernels of
// cf/vllm_tree/tree_ssm.py:60-62) and q scaled by Dk^-1/2.  State layout [H][Dk][Dv].
//
// Execution plan (path-parallel): one wave per (node, head, 64-column value slice).  Lane j owns
// state column j (all Dk = 128 rows) in registers and replays the node's ancestor chain from the
// root, so every node's state and output come from the same sequential per-path recurrence
// (tree_scan.py:78-90) and no wave waits for another.  q/k of each path step are normalised by the
// wave and broadcast through LDS.  The recompute costs depth x (3 Dk FMAs per lane) per node,
// which is far below the state traffic (S0 read, node state written).
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

__global__ void __launch_bounds__(64) k_gdn_tree(GdnArgs a) {
  __shared__ float qs[GDN_DK];
  __shared__ float ks[GDN_DK];
  __shared__ int path[GDN_MAXN];
  __shared__ int plen_s, bad_s;
  const int nvs = a.Dv / 64;
  int u = blockIdx.x;
  const int vs = u % nvs;
  u /= nvs;
  const int h = u % a.H;
  const int n = u / a.H;
  const int lane = threadIdx.x;
  const int j = vs * 64 + lane;

  if (lane == 0) {
    // ancestor chain n, parent(n), ..., root; indices strictly decrease, so at most n + 1 entries
    int len = 0, bad = 0, cur = n;
    while (true) {
      path[len++] = cur;
      const int p = a.parent[cur];
      if (p < 0) break;
      if (p >= cur) { bad = 1; break; }
      cur = p;
    }
    plen_s = len;
    bad_s = bad;
  }
  __syncthreads();
  const int len = plen_s;
  if (bad_s) {   // not BFS-ordered: refuse with NaN outputs rather than read a later node
    const float nan = __builtin_nanf("");
    a.out[((size_t)n * a.H + h) * a.Dv + j] = nan;
    if (a.states)
      for (int i = 0; i < GDN_DK; ++i) a.states[(((size_t)n * a.H + h) * GDN_DK + i) * a.Dv + j] = nan;
    return;
  }

  float S[GDN_DK];
  const float* s0 = a.S0 + (size_t)h * GDN_DK * a.Dv + j;
#pragma unroll
  for (int i = 0; i < GDN_DK; ++i) S[i] = s0[(size_t)i * a.Dv];

  float o = 0.f;
  for (int t = len - 1; t >= 0; --t) {
    const int m = path[t];
    const size_t qk = ((size_t)m * a.H + h) * GDN_DK;
    float q0 = bf16f(a.q[qk + lane]), q1 = bf16f(a.q[qk + 64 + lane]);
    float k0 = bf16f(a.k[qk + lane]), k1 = bf16f(a.k[qk + 64 + lane]);
    if (a.l2norm) {
      const float sq = wave_sum(q0 * q0 + q1 * q1);
      const float sk = wave_sum(k0 * k0 + k1 * k1);
      const float iq = a.l2mode ? 1.0f / sqrtf(sq + 1e-6f) : 1.0f / (sqrtf(sq) + 1e-6f);
      const float ik = a.l2mode ? 1.0f / sqrtf(sk + 1e-6f) : 1.0f / (sqrtf(sk) + 1e-6f);
      q0 *= iq; q1 *= iq; k0 *= ik; k1 *= ik;
    }
    __syncthreads();   // the previous step's reads of qs/ks are done
    qs[lane] = q0 * a.scale;
    qs[lane + 64] = q1 * a.scale;
    ks[lane] = k0;
    ks[lane + 64] = k1;
    __syncthreads();
    const float eg = expf(a.g[(size_t)m * a.H + h]);
    const float bt = a.beta[(size_t)m * a.H + h];
    const float vj = bf16f(a.v[((size_t)m * a.H + h) * a.Dv + j]);
    float kv = 0.f;
#pragma unroll
    for (int i = 0; i < GDN_DK; ++i) {
      S[i] *= eg;
      kv += S[i] * ks[i];
    }
    const float delta = (vj - kv) * bt;
    o = 0.f;
#pragma unroll
    for (int i = 0; i < GDN_DK; ++i) {
      S[i] += ks[i] * delta;
      o += S[i] * qs[i];
    }
  }
  a.out[((size_t)n * a.H + h) * a.Dv + j] = o;
  if (a.states) {
    float* st = a.states + ((size_t)n * a.H + h) * GDN_DK * a.Dv + j;
#pragma unroll
    for (int i = 0; i < GDN_DK; ++i) st[(size_t)i * a.Dv] = S[i];
  }
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
  hipLaunchKernelGGL(k_gdn_tree, dim3((unsigned)blocks), dim3(64), 0, (hipStream_t)stream, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

}  // extern "C"
