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
  int N, H, HV, V, ld, prefix, bf16_state, l2norm;
  float scale;
};

__device__ __forceinline__ float round_bf16(float x) {   // round to nearest even, as the cast does
  unsigned u = __float_as_uint(x);
  if ((u & 0x7f800000u) == 0x7f800000u) return x;        // inf / nan unchanged
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  return __uint_as_float(u);
}
__device__ __forceinline__ uint16_t to_bf16(float x) { return (uint16_t)(__float_as_uint(round_bf16(x)) >> 16); }

__global__ void __launch_bounds__(64) k_gdn_tree_vllm(GdnVArgs a) {
  __shared__ float qs[GDN_DK];
  __shared__ float ks[GDN_DK];
  __shared__ int path[GDN_MAXN];
  __shared__ int plen_s, bad_s;
  const int nvs = a.V / 64;
  int u = blockIdx.x;
  const int vs = u % nvs;
  u /= nvs;
  const int hv = u % a.HV;
  const int n = u / a.HV;
  const int h = hv / (a.HV / a.H);
  const int lane = threadIdx.x;
  const int j = vs * 64 + lane;
  const size_t srow = (size_t)a.HV * a.V * GDN_DK;                 // elements per slot
  const size_t sofs = ((size_t)hv * a.V + j) * GDN_DK;             // this lane's state row in a slot

  if (lane == 0) {
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
  if (bad_s) {   // not BFS-ordered: NaN outputs, state slot untouched
    a.out[((size_t)n * a.HV + hv) * a.V + j] = 0x7fc0;
    return;
  }

  float S[GDN_DK];
  if (a.bf16_state) {
    const uint16_t* s0 = (const uint16_t*)a.state + (size_t)a.prefix * srow + sofs;
#pragma unroll
    for (int i = 0; i < GDN_DK; ++i) S[i] = bf16f(s0[i]);
  } else {
    const float* s0 = (const float*)a.state + (size_t)a.prefix * srow + sofs;
#pragma unroll
    for (int i = 0; i < GDN_DK; ++i) S[i] = s0[i];
  }
  const float Aexp = expf(a.A_log[hv]), dtb = a.dt_bias[hv];
  const size_t koff = (size_t)a.H * GDN_DK + (size_t)h * GDN_DK;
  const size_t voff = 2 * (size_t)a.H * GDN_DK + (size_t)hv * a.V + j;
  for (int t = len - 1; t >= 0; --t) {
    const int m = path[t];
    const uint16_t* row = a.qkv + (size_t)m * a.ld;
    float k0 = bf16f(row[koff + lane]), k1 = bf16f(row[koff + 64 + lane]);
    if (a.l2norm) {
      const float ik = 1.0f / sqrtf(wave_sum(k0 * k0 + k1 * k1) + 1e-6f);
      k0 *= ik; k1 *= ik;
    }
    __syncthreads();   // the previous step's reads of ks are done
    ks[lane] = k0;
    ks[lane + 64] = k1;
    __syncthreads();
    const float x = bf16f(a.ga[(size_t)m * a.HV + hv]) + dtb;
    const float sp = x <= 20.0f ? logf(1.0f + expf(x)) : x;
    const float eg = expf(-Aexp * sp);
    const float bt = round_bf16(1.0f / (1.0f + expf(-bf16f(a.gb[(size_t)m * a.HV + hv]))));
    const float vj = bf16f(row[voff]);
    float kv = 0.f;
#pragma unroll
    for (int i = 0; i < GDN_DK; ++i) {
      S[i] *= eg;
      kv += S[i] * ks[i];
    }
    const float delta = (vj - kv) * bt;
#pragma unroll
    for (int i = 0; i < GDN_DK; ++i) S[i] += delta * ks[i];
    if (t > 0 && a.bf16_state) {   // an ancestor: its stored (bf16) state is what the child reads
#pragma unroll
      for (int i = 0; i < GDN_DK; ++i) S[i] = round_bf16(S[i]);
    }
  }
  // output with the node's own q
  const uint16_t* row = a.qkv + (size_t)n * a.ld;
  float q0 = bf16f(row[(size_t)h * GDN_DK + lane]), q1 = bf16f(row[(size_t)h * GDN_DK + 64 + lane]);
  if (a.l2norm) {
    const float iq = 1.0f / sqrtf(wave_sum(q0 * q0 + q1 * q1) + 1e-6f);
    q0 *= iq; q1 *= iq;
  }
  __syncthreads();
  qs[lane] = q0 * a.scale;
  qs[lane + 64] = q1 * a.scale;
  __syncthreads();
  float o = 0.f;
#pragma unroll
  for (int i = 0; i < GDN_DK; ++i) o += S[i] * qs[i];
  a.out[((size_t)n * a.HV + hv) * a.V + j] = to_bf16(o);
  const size_t dst = (size_t)a.slots[n] * srow + sofs;
  if (a.bf16_state) {
    uint16_t* st = (uint16_t*)a.state + dst;
#pragma unroll
    for (int i = 0; i < GDN_DK; ++i) st[i] = to_bf16(S[i]);
  } else {
    float* st = (float*)a.state + dst;
#pragma unroll
    for (int i = 0; i < GDN_DK; ++i) st[i] = S[i];
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

int cfh_gdn_tree_vllm(const void* mixed_qkv, const void* a, const void* b, const float* A_log, const float* dt_bias,
                      void* ssm_state, int state_bf16, const int32_t* node_slots, const int32_t* parent,
                      int prefix_slot, int N, int H, int HV, int K, int V, int use_l2norm, float scale,
                      void* out, void* stream) {
  if (!mixed_qkv || !a || !b || !A_log || !dt_bias || !ssm_state || !node_slots || !parent || !out)
    return CFH_E_INVALID;
  if (N < 1 || N > GDN_MAXN || H < 1 || HV < H || HV % H || V < 64 || V % 64 || prefix_slot < 0)
    return CFH_E_INVALID;
  if (K != GDN_DK) return CFH_E_UNSUPPORTED;
  GdnVArgs g = {};
  g.qkv = (const uint16_t*)mixed_qkv; g.ga = (const uint16_t*)a; g.gb = (const uint16_t*)b;
  g.A_log = A_log; g.dt_bias = dt_bias; g.state = ssm_state; g.slots = node_slots; g.parent = parent;
  g.out = (uint16_t*)out; g.N = N; g.H = H; g.HV = HV; g.V = V; g.ld = 2 * H * K + HV * V;
  g.prefix = prefix_slot; g.bf16_state = state_bf16 ? 1 : 0; g.l2norm = use_l2norm ? 1 : 0; g.scale = scale;
  const long long blocks = (long long)N * HV * (V / 64);
  hipLaunchKernelGGL(k_gdn_tree_vllm, dim3((unsigned)blocks), dim3(64), 0, (hipStream_t)stream, g);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

}  // extern "C"
