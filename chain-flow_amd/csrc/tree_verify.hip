// The rest of the tree verify on MI355X (the forked vLLM's tree arm):
//   * tree causal conv1d of the GDN layers (cf/vllm_tree/tree_ssm.py:393-438; depth form :189-253);
//   * the ancestor-masked attention of the draft-tree rows plus the log-sum-exp merge with the
//     shared-prefix attention (patch _tree_attention_fixup / _tree_suffix_eager, lines 403-575;
//     the fused CUDA form tree_attn_fused.cu, 5095-5540);
//   * the greedy tree descent that accepts the longest draft path the target agrees with
//     (patch tree_greedy_descent_kernel / tree_rejection_sample, lines 433-550).
#include <math.h>

#include "cfh_kernels.h"

namespace {

typedef unsigned short u16;

__device__ __forceinline__ float bf2f(u16 b) { return __uint_as_float((unsigned)b << 16); }
__device__ __forceinline__ u16 f2bf(float f) {   // round to nearest even (NaN kept quiet)
  const unsigned u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u16)((u >> 16) | 0x40);
  return (u16)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// 2-byte element types: bf16 (IS_BF16) or fp16
template <bool IS_BF16>
__device__ __forceinline__ float ld2(const u16* p, size_t i) {
  if constexpr (IS_BF16) return bf2f(p[i]);
  else return (float)__builtin_bit_cast(_Float16, p[i]);
}
template <bool IS_BF16>
__device__ __forceinline__ u16 cv2(float f) {
  if constexpr (IS_BF16) return f2bf(f);
  else return __builtin_bit_cast(u16, (_Float16)f);
}
template <bool IS_BF16>
__device__ __forceinline__ float rt2(float f) {   // round to the 2-byte type and back
  if constexpr (IS_BF16) return rbf(f);
  else return (float)(_Float16)f;
}

// ---------------------------------------------------------------------------- tree conv1d
// Width-4 causal conv over the tree, bf16 storage: the state of a node is the last three inputs
// along its root->node path (the prefix slot's state before the root) plus the prefix slot's
// fourth column carried unchanged; out = act(bias + bf16(s0 w0) + bf16(s1 w1) + bf16(s2 w2) +
// bf16(x w3)) with bf16 products summed in fp32 left to right (tree_ssm.py:406-414), act = SiLU or
// none, and the node's state (s1, s2, x, s3) is written to its slot.  One thread per (node,
// feature): a node's window is read off its (at most three) ancestors' inputs directly, so every
// node runs in parallel and gives what the node-serial form gives.
struct ConvArgs {
  const u16* x;          // [N][x_ld] bf16
  u16* state;            // [slots][dim][4] bf16
  const u16* w;          // [dim][4] bf16
  const u16* bias;       // [dim] bf16 or null
  u16* out;              // [N][out_ld] bf16
  const int* node_slots; // [N]
  const int* parent;     // [N] node index, -1 = root
  int prefix_slot, N, dim, x_ld, out_ld, silu;
};

__global__ void __launch_bounds__(256) k_tree_conv(ConvArgs a) {
  const int f = blockIdx.x * blockDim.x + threadIdx.x;
  const int n = blockIdx.y;
  if (f >= a.dim) return;
  const u16* ps = a.state + ((size_t)a.prefix_slot * a.dim + f) * 4;
  // the input sequence seen by the node: [p0 p1 p2 | x(a_k) .. x(a_1)], a_1 = the parent, k <= 3
  // nearest ancestors; its last three entries are the window
  u16 win[6];
  win[0] = ps[0]; win[1] = ps[1]; win[2] = ps[2];
  const u16 p3 = ps[3];
  int anc[3], k = 0;
  for (int m = a.parent[n]; m >= 0 && k < 3; m = a.parent[m]) anc[k++] = m;
  for (int i = 0; i < k; ++i) win[3 + (k - 1 - i)] = a.x[(size_t)anc[i] * a.x_ld + f];
  const u16 s0 = win[k], s1 = win[k + 1], s2 = win[k + 2];
  const u16 xi = a.x[(size_t)n * a.x_ld + f];
  const u16* w = a.w + (size_t)f * 4;
  float acc = a.bias ? bf2f(a.bias[f]) : 0.f;
  acc = acc + rbf(bf2f(s0) * bf2f(w[0]));
  acc = acc + rbf(bf2f(s1) * bf2f(w[1]));
  acc = acc + rbf(bf2f(s2) * bf2f(w[2]));
  acc = acc + rbf(bf2f(xi) * bf2f(w[3]));
  if (a.silu) acc = acc * (1.0f / (1.0f + expf(-acc)));
  a.out[(size_t)n * a.out_ld + f] = f2bf(acc);
  u16* ns = a.state + ((size_t)a.node_slots[n] * a.dim + f) * 4;
  ns[0] = s1; ns[1] = s2; ns[2] = xi; ns[3] = p3;
}

// ---------------------------------------------------------------------------- tree attention
// For request s, tree node n and head h (query row idx[s][n]): scores over the nodes m the mask
// allows (ancestors and the node itself), scale * q.k in fp32; softmax with the max and the
// denominator summed over those columns in order; lse_s = max + log(denom); the weighted sum of v
// in fp32, rounded to the output type; then the merge with the prefix half (vLLM's
// merge_attn_states): m = max(lse_p, lse_s) (inf -> -inf), e_p = exp(lse_p - m), e_s = exp(lse_s
// - m), out = fma(p_out, e_p / (e_p + e_s), s_out * (e_s / (e_p + e_s))).  Grouped heads: head h
// reads kv head h / (H / Hkv).  One wave per (s, n, h); lane l owns head-dim elements l*EPL ..
// (D = 64 EPL).  Masked columns contribute exactly nothing (exp(-inf) = 0), so they are skipped.
struct AttnArgs {
  const u16* q; const u16* k; const u16* v;   // rows of the forward: [T][H|Hkv][D]
  u16* out;                                   // [T][H][D]: tree rows written in place
  const u16* pout;                            // [S*N][H][D] prefix half, compact tree order
  const float* plse;                          // [H][S*N]
  const int* idx;                             // [S][N] forward row of each tree node
  const unsigned char* not_anc;               // [S][N][N] 1 = masked
  float scale;
  int S, N, H, Hkv, q_ld, k_ld, v_ld, o_ld;   // row strides in elements
};

constexpr int TA_WAVES = 4;
constexpr int TA_NMAX = 128;

// 2-byte elements of one lane, loaded as one vector
template <int EPL> struct LaneVec;
template <> struct LaneVec<1> { typedef u16 type; };
template <> struct LaneVec<2> { typedef unsigned type; };
template <> struct LaneVec<4> { typedef uint2 type; };

template <bool IS_BF16, int EPL>
__device__ __forceinline__ void widen(const typename LaneVec<EPL>::type& r, float (&o)[EPL]) {
  const u16* t = (const u16*)&r;
#pragma unroll
  for (int e = 0; e < EPL; ++e) o[e] = ld2<IS_BF16>(t, e);
}

constexpr int TA_BATCH = 8;   // key / value rows whose loads are in flight together

// The unmasked columns of the row, lowest first, as two wave-uniform 64-bit sets.
struct ColSet {
  unsigned long long lo, hi;
  __device__ __forceinline__ bool empty() const { return !(lo | hi); }
  __device__ __forceinline__ int pop() {
    if (lo) { const int m = __builtin_ctzll(lo); lo &= lo - 1; return m; }
    const int m = 64 + __builtin_ctzll(hi); hi &= hi - 1; return m;
  }
};

template <bool IS_BF16, int EPL>
__global__ void __launch_bounds__(TA_WAVES * 64) k_tree_attn(AttnArgs a) {
  typedef typename LaneVec<EPL>::type VT;
  __shared__ float sc[TA_WAVES][TA_NMAX];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int gw = blockIdx.x * TA_WAVES + wave;
  if (gw >= a.S * a.N * a.H) return;
  const int h = gw % a.H;
  const int sn = gw / a.H;
  const int s = sn / a.N, n = sn - s * a.N;
  const int hk = h / (a.H / a.Hkv);
  const int D = 64 * EPL;
  const int* idx = a.idx + (size_t)s * a.N;
  const unsigned char* mask = a.not_anc + ((size_t)s * a.N + n) * a.N;
  const int row = s * a.N + n;
  // round trip 1, every independent load: the mask row and the request's row indices (one column
  // per lane), q, the prefix half
  const int c0 = min(lane, a.N - 1), c1 = min(64 + lane, a.N - 1);
  const bool ok0 = lane < a.N && !mask[c0];
  const bool ok1 = 64 + lane < a.N && !mask[c1];
  const int ix0 = idx[c0], ix1 = idx[c1];
  const VT qraw = *(const VT*)(a.q + (size_t)idx[n] * a.q_ld + (size_t)h * D + lane * EPL);
  const VT praw = *(const VT*)(a.pout + ((size_t)row * a.H + h) * D + lane * EPL);
  float lp = a.plse[(size_t)h * a.S * a.N + row];
  ColSet cs = {__ballot(ok0), __ballot(ok1)};
  auto row_of = [&](int m) { return m < 64 ? __builtin_amdgcn_readlane(ix0, m) : __builtin_amdgcn_readlane(ix1, m - 64); };
  float qv[EPL];
  widen<IS_BF16, EPL>(qraw, qv);
  // round trip 2 (per TA_BATCH columns): the key AND value rows of the unmasked columns together;
  // the scores go to LDS (column ordinal order), then the max, the denominator and the weighted
  // sum follow in increasing column order
  float mx = -INFINITY, den = 0.f;
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  int ncol = 0;
  while (!cs.empty()) {
    int ms[TA_BATCH];
    VT kr[TA_BATCH], vr[TA_BATCH];
    int cnt = 0;
#pragma unroll
    for (int c = 0; c < TA_BATCH; ++c) {
      ms[c] = cs.empty() ? -1 : cs.pop();
      if (ms[c] >= 0) ++cnt;
      const size_t rr = (size_t)row_of(max(ms[c], 0));
      kr[c] = *(const VT*)(a.k + rr * a.k_ld + (size_t)hk * D + lane * EPL);
      vr[c] = *(const VT*)(a.v + rr * a.v_ld + (size_t)hk * D + lane * EPL);
    }
#pragma unroll
    for (int c = 0; c < TA_BATCH; ++c) {
      if (c >= cnt) break;
      float kv[EPL];
      widen<IS_BF16, EPL>(kr[c], kv);
      float part = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) part += qv[e] * kv[e];
      // the wave total is the same in every lane: each lane stores it and later reads back its own
      const float sm = wave_sum(part) * a.scale;
      sc[wave][ncol + c] = sm;
      mx = fmaxf(mx, sm);
    }
    ncol += cnt;
    // keep the value rows of this batch in registers for the weighted sum below only when every
    // column fits one batch (the common tree: depth + 1 <= TA_BATCH ancestors)
    if (cs.empty() && ncol == cnt) {
      for (int c = 0; c < cnt; ++c) den += expf(sc[wave][c] - mx);
#pragma unroll
      for (int c = 0; c < TA_BATCH; ++c) {
        if (c >= cnt) break;
        const float p = expf(sc[wave][c] - mx) / den;
        float vv[EPL];
        widen<IS_BF16, EPL>(vr[c], vv);
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] += p * vv[e];
      }
      ncol = -1;   // done
    }
  }
  if (ncol >= 0) {
    // more than one batch of columns: the denominator, then a second pass over the value rows
    for (int c = 0; c < ncol; ++c) den += expf(sc[wave][c] - mx);
    ColSet cv = {__ballot(ok0), __ballot(ok1)};
    int c = 0;
    while (!cv.empty()) {
      int ms[TA_BATCH];
      VT vr[TA_BATCH];
      int cnt = 0;
#pragma unroll
      for (int u = 0; u < TA_BATCH; ++u) {
        ms[u] = cv.empty() ? -1 : cv.pop();
        if (ms[u] >= 0) ++cnt;
        vr[u] = *(const VT*)(a.v + (size_t)row_of(max(ms[u], 0)) * a.v_ld + (size_t)hk * D + lane * EPL);
      }
#pragma unroll
      for (int u = 0; u < TA_BATCH; ++u) {
        if (u >= cnt) break;
        const float p = expf(sc[wave][c + u] - mx) / den;
        float vv[EPL];
        widen<IS_BF16, EPL>(vr[u], vv);
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] += p * vv[e];
      }
      c += cnt;
    }
  }
  const float lse_s = mx + logf(den);
  float ls = lse_s;
  if (isinf(lp)) lp = -INFINITY;
  if (isinf(ls)) ls = -INFINITY;
  const float mm = fmaxf(lp, ls);
  const float ep = expf(lp - mm), es = expf(ls - mm);
  const float tot = ep + es;
  const float psc = ep / tot, ssc = es / tot;
  float pv[EPL];
  widen<IS_BF16, EPL>(praw, pv);
  VT ov;
  u16* ot = (u16*)&ov;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float so = rt2<IS_BF16>(acc[e]);   // the suffix half is handed over in the output type
    ot[e] = cv2<IS_BF16>(fmaf(pv[e], psc, so * ssc));
  }
  *(VT*)(a.out + (size_t)idx[n] * a.o_ld + (size_t)h * D + lane * EPL) = ov;
}

// ---------------------------------------------------------------------------- greedy descent
// row_argmax[r] = first index of the maximum of logits row r (torch.argmax), in two steps:
// ACC_SPLIT workgroups per row each scan a slice with 16-byte loads (8 elements a lane) keeping
// (value, first index), reduced over the wave and the workgroup (the larger value, then the lower
// index) into ws[r][split]; the descent kernel then reduces a request's rows' slices in slice order.
constexpr int ACC_SPLIT = 16;

struct ArgPart { float v; int i; };

__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

template <bool IS_BF16, bool VEC>
__global__ void __launch_bounds__(256) k_argmax_part(const u16* logits, int V, long long ld, ArgPart* ws) {
  __shared__ float bv[4];
  __shared__ int bi[4];
  const u16* row = logits + (size_t)blockIdx.x * ld;
  const int per = (V + ACC_SPLIT - 1) / ACC_SPLIT;
  const int c0 = blockIdx.y * per, c1 = min(V, c0 + per);
  float best = -INFINITY;
  int bix = V;
  if constexpr (VEC) {
    // 8-element vectors over the aligned middle of [c0, c1), scalars at both ends
    const int v0 = (c0 + 7) / 8, v1 = c1 / 8;
    for (int j = c0 + threadIdx.x; j < min(c1, v0 * 8); j += blockDim.x) better(best, bix, ld2<IS_BF16>(row, j), j);
    for (int u = v0 + threadIdx.x; u < v1; u += blockDim.x) {
      const uint4 raw = *(const uint4*)(row + (size_t)u * 8);
      const u16* t = (const u16*)&raw;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = ld2<IS_BF16>(t, e);
        if (v > best) { best = v; bix = u * 8 + e; }   // increasing index within a thread: > keeps the first
      }
    }
    for (int j = max(v1 * 8, v0 * 8) + threadIdx.x; j < c1; j += blockDim.x) better(best, bix, ld2<IS_BF16>(row, j), j);
  } else {
    for (int j = c0 + threadIdx.x; j < c1; j += blockDim.x) better(best, bix, ld2<IS_BF16>(row, j), j);
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best, off);
    const int oi = __shfl_xor(bix, off);
    better(best, bix, ov, oi);
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) { bv[wave] = best; bi[wave] = bix; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) better(best, bix, bv[w], bi[w]);
    ws[(size_t)blockIdx.x * ACC_SPLIT + blockIdx.y] = ArgPart{best, bix};
  }
}

// Per request r (one workgroup): its rows s0 .. s0 + n of the flat logits (row 0 = the last
// committed token, row 1 + i = tree node i) get their arg-max from the slices; then the wave
// walks the tree: from the root row, emit the target's token at the current row; move to the first
// child whose draft token equals it (64 nodes tested at a time, a ballot picks the lowest); stop
// when none does.  Output tokens (accepted drafts + the
// bonus) [B][max_spec + 1] (-1 padded), accepted path (node per depth, -1 padded) [B][max_spec],
// accepted length [B].
struct DescentArgs {
  const int* cu_draft;     // [B] inclusive cumulative draft tokens
  const int* cu_sampled;   // [B] inclusive cumulative rows (draft tokens + 1)
  const int* draft;        // [total drafts] token ids
  const int* parents;      // [total drafts] local parent node, -1 = root
  const ArgPart* ws;       // [rows][ACC_SPLIT]
  int* row_argmax;         // [rows]
  int* out_tokens;
  int* path;
  int* len;
  int B, max_spec, V;
};

constexpr int ACC_LDS = 1024;   // draft nodes per request staged in LDS for the walk

__global__ void __launch_bounds__(64) k_tree_descent(DescentArgs a) {
  __shared__ int s_par[ACC_LDS], s_tok[ACC_LDS], s_arg[ACC_LDS + 1];
  const int r = blockIdx.x;
  const int d0 = r == 0 ? 0 : a.cu_draft[r - 1], n = a.cu_draft[r] - d0;
  const int s0 = a.cu_sampled[r] - (n + 1);
  const bool lds = n <= ACC_LDS;
  for (int j = threadIdx.x; j <= n; j += blockDim.x) {
    const ArgPart* p = a.ws + (size_t)(s0 + j) * ACC_SPLIT;
    float bv = -INFINITY;
    int bi = a.V;
    for (int k = 0; k < ACC_SPLIT; ++k) better(bv, bi, p[k].v, p[k].i);
    bi = bi < a.V ? bi : 0;
    a.row_argmax[s0 + j] = bi;
    if (lds) s_arg[j] = bi;
    if (lds && j < n) {
      s_par[j] = a.parents[d0 + j];
      s_tok[j] = a.draft[d0 + j];
    }
  }
  int* ot = a.out_tokens + (size_t)r * (a.max_spec + 1);
  int* pt = a.path + (size_t)r * a.max_spec;
  for (int i = threadIdx.x; i <= a.max_spec; i += blockDim.x) ot[i] = -1;
  for (int i = threadIdx.x; i < a.max_spec; i += blockDim.x) pt[i] = -1;
  __syncthreads();
  // the walk: at each level the wave tests 64 nodes at a time for (parent == cur, token == the
  // row's argmax); the lowest matching index is the first child in draft order
  const int lane = threadIdx.x;
  int cur = -1, pos = 0;
  for (int step = 0; step <= a.max_spec; ++step) {
    const int tok = lds ? s_arg[cur + 1] : a.row_argmax[s0 + cur + 1];
    if (lane == 0) ot[pos] = tok;
    int nxt = -1;
    if (pos < a.max_spec) {
      for (int i0 = 0; i0 < n; i0 += 64) {
        const int i = i0 + lane;
        bool hit = false;
        if (i < n) {
          const int pi = lds ? s_par[i] : a.parents[d0 + i];
          const int ti = lds ? s_tok[i] : a.draft[d0 + i];
          hit = pi == cur && ti == tok;
        }
        const unsigned long long m = __ballot(hit);
        if (m) {
          nxt = i0 + __ffsll((long long)m) - 1;
          break;
        }
      }
    }
    if (nxt < 0) break;
    if (lane == 0) pt[pos] = nxt;
    cur = nxt;
    ++pos;
  }
  if (lane == 0) a.len[r] = pos;
}

}  // namespace

extern "C" {

int cfh_tree_conv(const void* x, int x_ld, void* conv_state, const void* weight, const void* bias,
                  const int32_t* node_slots, const int32_t* parent, int prefix_slot, int N, int dim, int silu,
                  void* out, int out_ld, void* stream) {
  if (N == 0) return CFH_OK;
  if (!x || !conv_state || !weight || !node_slots || !parent || !out || N < 0 || dim <= 0 || x_ld < dim ||
      out_ld < dim || prefix_slot < 0)
    return CFH_E_INVALID;
  if (N > 65535) return CFH_E_UNSUPPORTED;
  ConvArgs a = {(const u16*)x, (u16*)conv_state, (const u16*)weight, (const u16*)bias, (u16*)out, node_slots,
                parent, prefix_slot, N, dim, x_ld, out_ld, silu};
  hipLaunchKernelGGL(k_tree_conv, dim3((dim + 255) / 256, N), dim3(256), 0, (hipStream_t)stream, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int cfh_tree_attn_merge(const void* q, int q_ld, const void* k, int k_ld, const void* v, int v_ld, void* out,
                        int o_ld, const void* prefix_out, const float* prefix_lse, const int32_t* idx,
                        const uint8_t* not_anc, float scale, int S, int N, int H, int Hkv, int D, int is_bf16,
                        void* stream) {
  if (S == 0 || N == 0) return CFH_OK;
  if (!q || !k || !v || !out || !prefix_out || !prefix_lse || !idx || !not_anc || S < 0 || N < 0 || H <= 0 ||
      Hkv <= 0 || H % Hkv)
    return CFH_E_INVALID;
  if (N > TA_NMAX || (D != 64 && D != 128 && D != 256)) return CFH_E_UNSUPPORTED;
  // each lane loads D / 64 elements as one vector
  const int vb = D / 32;   // bytes per lane
  for (const void* ptr : {q, k, v, (const void*)out, prefix_out})
    if ((uintptr_t)ptr % vb) return CFH_E_INVALID;
  if ((q_ld * 2) % vb || (k_ld * 2) % vb || (v_ld * 2) % vb || (o_ld * 2) % vb) return CFH_E_INVALID;
  AttnArgs a = {(const u16*)q, (const u16*)k, (const u16*)v, (u16*)out, (const u16*)prefix_out, prefix_lse, idx,
                not_anc, scale, S, N, H, Hkv, q_ld, k_ld, v_ld, o_ld};
  const long long waves = (long long)S * N * H;
  const dim3 grid((unsigned)((waves + TA_WAVES - 1) / TA_WAVES)), block(TA_WAVES * 64);
  hipStream_t st = (hipStream_t)stream;
#define CFH_TA(BF, E) hipLaunchKernelGGL((k_tree_attn<BF, E>), grid, block, 0, st, a)
  if (is_bf16) {
    if (D == 64) CFH_TA(true, 1); else if (D == 128) CFH_TA(true, 2); else CFH_TA(true, 4);
  } else {
    if (D == 64) CFH_TA(false, 1); else if (D == 128) CFH_TA(false, 2); else CFH_TA(false, 4);
  }
#undef CFH_TA
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int64_t cfh_tree_accept_ws_bytes(int n_rows) {
  if (n_rows < 0) return -1;
  return (int64_t)n_rows * ACC_SPLIT * (int64_t)sizeof(ArgPart);
}

int cfh_tree_greedy_accept(const void* logits, long long ld, int V, int n_rows, int is_bf16, const int32_t* cu_draft,
                           const int32_t* cu_sampled, const int32_t* draft_ids, const int32_t* parents, int B,
                           int max_spec, int32_t* out_tokens, int32_t* accepted_path, int32_t* accepted_len,
                           int32_t* row_argmax, void* ws, void* stream) {
  if (B == 0) return CFH_OK;
  if (!logits || !cu_draft || !cu_sampled || !out_tokens || !accepted_path || !accepted_len || !row_argmax || !ws ||
      V <= 0 || n_rows <= 0 || B < 0 || max_spec < 0 || ld < V)
    return CFH_E_INVALID;
  hipStream_t st = (hipStream_t)stream;
  const bool vec = ld % 8 == 0 && ((uintptr_t)logits & 15) == 0;
  const dim3 grid(n_rows, ACC_SPLIT);
  const u16* lg = (const u16*)logits;
  ArgPart* w = (ArgPart*)ws;
  if (is_bf16) {
    if (vec) hipLaunchKernelGGL((k_argmax_part<true, true>), grid, dim3(256), 0, st, lg, V, ld, w);
    else hipLaunchKernelGGL((k_argmax_part<true, false>), grid, dim3(256), 0, st, lg, V, ld, w);
  } else {
    if (vec) hipLaunchKernelGGL((k_argmax_part<false, true>), grid, dim3(256), 0, st, lg, V, ld, w);
    else hipLaunchKernelGGL((k_argmax_part<false, false>), grid, dim3(256), 0, st, lg, V, ld, w);
  }
  CFH_LAUNCH_CHECK();
  DescentArgs a = {cu_draft, cu_sampled, draft_ids, parents, w, row_argmax, out_tokens, accepted_path, accepted_len,
                   B, max_spec, V};
  hipLaunchKernelGGL(k_tree_descent, dim3(B), dim3(64), 0, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

}  // extern "C"
