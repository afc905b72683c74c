// The chain-flow velocity net + Euler integrator on MI355X: TreeFlowDrafter.predict_hidden.
//
// Reference semantics (cf/ = src/chain_flow/): init_latents cf/drafters/tree_flow.py:150-161,
// integrate :229-235, flow_velocity/_chunk_args :163-190, HiddenKVFlowExpert.pre_blocks /
// post_blocks cf/drafters/chunked_flow.py:333-384, HiddenKVFlowBlock.forward :185-202; fused-kernel
// numerics cf/csrc/fused_block.cu:280-325, 452-668, 674-722 (fp32 residual, fp16-parked LayerNorm
// rows, fp16 q/k/v, attention and GELU outputs, cross K/V hoisted once per draft).
//
// Numerics: the fused kernel's (fp32 residual x += sublayer; GELU of the fp32 pre-activation) or
// torch's fp16 modules' (x = fp16(x + fp16(sublayer)); GELU of the fp16-rounded up-projection), as
// cfh_flow_dims.numerics says; only the residual row kernel and the W1 epilogue differ.
//
// Execution plan.  One launch sequence per group of requests.  The per-draft launches cover every
// chunk expert at once; then each expert runs its Euler steps on its own stream (the caller's, then
// companion streams), and one expert's row kernels and launch gaps overlap another's weight
// streaming.  Within a step the experts are independent; expert c's next rows read the rows of the
// chunks before c as the step left them (tree_flow.py _chunk_args), so only its Euler update waits
// for theirs (and an expert's next update waits until the next expert has read its chunk's rows).
// A batch is drafted in groups of R requests whose rows share one MFMA tile (R x draft_length
// <= 16: two 8-row drafts, where the 16-row operand fits the streaming kernels' LDS: d <= 4096 of
// the supported widths), so every weight stream serves R drafts; attention masks keep each request
// to its own rows and context.  Work that needs a whole row sits in a small row kernel between two
// streaming kernels; there is no cross-workgroup synchronisation inside any kernel (no fences, no
// atomics, no spin-waits), so results are deterministic.  On MI355X the gap between two kernels on the stream is 1.4-2 us (per-workgroup
// timestamps), while a fenced grid barrier across the 8 XCDs costs ~12 us, which is why this is a
// kernel pipeline and not one persistent launch.
//
//   per expert: TAU  time_mlp(tau_s) for all E steps, computed when the expert is packed
//   per draft : ROWS init_latents(ctx), step-0 rows x, a = LN_self(x) of block 0
//               KV   cross K/V of every block             (GEMV + reduce)
//               FOLD A_h = Wq_h^T K_h^T, B_h = Wo_h V_h of every block (stream, split-K by head;
//                    several blocks a launch at narrow widths)
//   per Euler step, per block l (each expert on its own stream, the second starting ~1/3 block later):
//     QKV   stream  A = a (LN_self rows)          epilogue q,k,v = fp16(acc + b)      full-K tiles
//     O     stream  A = causal self attention of head h, computed while staging    split-K by head
//     RES   row     x += sum_h P + b_o ; a = LN_cross(fp16(x))
//     XATT  small   scores_h = a A_h + bq_h K_h^T, softmax, P_h B_h per head (fp32 partials)
//     RES   row     x += sum_h P + b_oc ; a = LN_ffn(fp16(x))
//           (one-request flows of width <= 640: RES, XATT, RES as one XBLK launch)
//     W1    stream  A = a                         epilogue g = fp16(gelu(acc + b1))  full-K tiles
//     W2    stream  A = g                         fp32 partials                     split-K
//     RES   row     x += sum P + b2 ; a = LN_self of block l+1 (out_norm after the last block)
//   OUT   stream  A = out_norm rows of the current chunk                           split-K
//   ROWS  row     v = fp16(sum P + b_out); z = fp16(z + fp16(dt v)); next step's rows and LN_self
//                 (per expert: its chunk's update and its own rows)
//
// The cross attention's query and output projections are folded into the context: the context is
// fixed for the whole draft, so q_h . K_h = LN(x) . (Wq_h^T K_h^T) + bq_h . K_h and
// Wo (P V) = sum_h P_h (Wo_h V_h); the two d x (H C) factors are built once per draft from Wq and
// Wo, and no block pass streams those two d x d matrices again (2 d^2 of the 18 d^2 halves a block
// pass reads).  Same products in exact arithmetic; q and the attention output are not rounded to
// fp16 on the way.  With two heads per MFMA k-chunk (head widths such as 80 or 240) one k-chunk's
// operand holds the context rows twice, each copy masked to one of its heads, so one weight stream
// still yields every head's factor apart (single-request groups: 2 C rows fill the 16-row tile;
// packed groups keep the unfolded QC / OC launches, and the packed image holds Wq both ways).
// Four heads per k-chunk keep the unfolded launches.
//
#include <stdio.h>

#include <algorithm>
#include <map>
#include <mutex>

#include "cfh_wide.h"

namespace {

// ROWS: one workgroup per z row r.
//   init  : z[r] = init_latents(ctx)[r] (delta mode, fp16 arithmetic); context row moments
//   euler : v = fp16(sum_kc Pout[kc][i] + b_out) for the chunk c, row i owning z row r;
//           z[r] = fp16(z[r] + fp16(dt v))   (z_out[r] = z[r] after the last step)
// then, unless this was the last step, the next step's rows: for every expert c2 that reads z row
// r: x = fp16(fp16(z + pos[r]) + [current rows] tau), residual x = that, a = LN_self of block 0.
// With `only` = c (each expert on its own stream) the launch updates chunk c's rows and builds
// expert c's rows alone, reading the earlier chunks' rows from z.
struct RowsArgs {
  const h16* ctx;      // [R][C][d] context rows of the group's requests
  float* ctx_mom;      // init: [R C][2] (mean, rstd) of the fp16 context rows
  float* z;            // [R][KD][d]
  h16* z_out;          // [R][KD][d]
  const float* Pout[4];
  const h16* bout[4];
  float* x[4];
  const h16* pos[4];
  const h16* tau[4];
  const h16* g[4];
  const h16* b[4];
  h16* a[4];
  float dt;
  int euler, last, ks, d, C, CS, nch, KD;
  int R;               // requests in the group (row r of the grid: request r / KD, draft row r % KD)
  int out_all;         // the OUT launch covered every row of each expert (R > 1), not just the current chunk's
  int init;            // CFH_INIT_*: how z0 is formed
  int only;            // euler: -1 = every chunk; c = chunk c's update and expert c's next rows only
                       // (the rows of earlier chunks are read from z, already updated)
  const h16* anchor[4];  // per expert, the group's anchor rows [R][d] (the anchored latent drafter), or null
};

template <int RQ>   // float4 groups a thread: d / 4 <= RQ * ROWT
__global__ void __launch_bounds__(ROWT) k_rows(RowsArgs a) {
  __shared__ float red[ROWT / 64];
  const int r = blockIdx.x, d = a.d, nq = d / 4;
  const int req = r / a.KD, rr = r - req * a.KD;
  float4 zv[RQ];
  h16x4 pp4[RQ], tt4[RQ];   // position and time rows of expert c2pre's next rows, loaded up front
  int c2pre = -1;
  if (!a.euler) {
    // moments of context rows r, r + gridDim.x, ... (read by the cross K/V GEMV)
    for (int cr = r; cr < a.R * a.C; cr += gridDim.x) {
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
    const h16* last = a.ctx + (size_t)(req * a.C + a.C - 1) * d;
    const h16* prev = a.ctx + (size_t)(req * a.C + a.C - 2) * d;
    const h16* given = a.z_out + (size_t)r * d;
    const float step = (float)(rr + 1);
#pragma unroll
    for (int k = 0; k < RQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      zv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (q < nq) {
        float o[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float lv = (float)last[q * 4 + t];
          if (a.init == CFH_INIT_GIVEN) {
            o[t] = (float)given[q * 4 + t];
          } else if (a.init == CFH_INIT_REPEAT_LAST) {
            o[t] = lv;
          } else {
            const float delta = r16(lv - (float)prev[q * 4 + t]);
            o[t] = r16(lv + r16(step * delta));
          }
        }
        zv[k] = make_float4(o[0], o[1], o[2], o[3]);
        *(float4*)(a.z + (size_t)r * d + q * 4) = zv[k];
      }
    }
  } else if (a.only >= 0 && rr / a.CS != a.only) {
    // a row of another chunk: past chunk `only`, no row of its expert; before it, read the row
    // that chunk's own update wrote for the next step's rows
    if (a.last || rr / a.CS > a.only) return;
#pragma unroll
    for (int k = 0; k < RQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      zv[k] = q < nq ? *(const float4*)(a.z + (size_t)r * d + q * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  } else {
    const int c = rr / a.CS, i = rr - c * a.CS;
    const int Sc = (c + 1) * a.CS;
    const size_t pst = (size_t)(a.out_all ? a.R * Sc : a.CS) * d;
    const float* Pr = a.Pout[c] + (size_t)(a.out_all ? req * Sc + c * a.CS + i : i) * d;
    // every load of the row in one batch: the out_proj partials, z, b_out and, unless this is the
    // last step, the position and time rows of expert c's next rows (the first expert that reads
    // this row), instead of a chain of dependent round trips
    if (!a.last) c2pre = c;
    float4 acc[RQ], zo[RQ];
    h16x4 bo4[RQ];
#pragma unroll
    for (int k = 0; k < RQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      if (q < nq) {
        acc[k] = *(const float4*)(Pr + q * 4);
        zo[k] = *(const float4*)(a.z + (size_t)r * d + q * 4);
        bo4[k] = *(const h16x4*)(a.bout[c] + q * 4);
        if (c2pre >= 0) {
          pp4[k] = *(const h16x4*)(a.pos[c] + (size_t)rr * d + q * 4);
          tt4[k] = *(const h16x4*)(a.tau[c] + q * 4);
        }
      }
    }
    constexpr int PB = RQ <= 2 ? 4 : 2;   // partial rows a batch (registers)
    for (int kc = 1; kc < a.ks; kc += PB) {
      float4 t[PB][RQ];
#pragma unroll
      for (int u = 0; u < PB; ++u)
#pragma unroll
        for (int k = 0; k < RQ; ++k) {
          const int q = threadIdx.x + k * blockDim.x;
          t[u][k] = (q < nq && kc + u < a.ks) ? *(const float4*)(Pr + (kc + u) * pst + q * 4)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
      for (int u = 0; u < PB; ++u)
#pragma unroll
        for (int k = 0; k < RQ; ++k)
          if (kc + u < a.ks) { acc[k].x += t[u][k].x; acc[k].y += t[u][k].y; acc[k].z += t[u][k].z; acc[k].w += t[u][k].w; }
    }
#pragma unroll
    for (int k = 0; k < RQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      zv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (q < nq) {
        const h16x4 bo = bo4[k];
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
  for (int c2 = a.only >= 0 ? a.only : 0; c2 < (a.only >= 0 ? a.only + 1 : a.nch); ++c2) {
    if (rr >= (c2 + 1) * a.CS) continue;         // expert c2 reads z rows [0, (c2+1)*CS) of each draft
    const bool cur = rr >= c2 * a.CS;
    const size_t xr = (size_t)req * (c2 + 1) * a.CS + rr;   // the row in expert c2's request-major rows
    float4 vals[RQ];
#pragma unroll
    for (int k = 0; k < RQ; ++k) {
      const int q = threadIdx.x + k * blockDim.x;
      vals[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (q < nq) {
        h16x4 pp, tt;
        if (c2 == c2pre) {
          pp = pp4[k];
          tt = tt4[k];
        } else {
          pp = *(const h16x4*)(a.pos[c2] + (size_t)rr * d + q * 4);
          tt = *(const h16x4*)(a.tau[c2] + q * 4);
        }
        const h16* an = a.anchor[c2] ? a.anchor[c2] + (size_t)req * d + q * 4 : nullptr;
        float o[4] = {zv[k].x, zv[k].y, zv[k].z, zv[k].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float xv = r16(o[t] + (float)pp[t]);
          if (cur) xv = r16(xv + (float)tt[t]);
          if (an) xv = r16(xv + (float)an[t]);   // the anchor conditions every row of every block
          o[t] = xv;
        }
        vals[k] = make_float4(o[0], o[1], o[2], o[3]);
        *(float4*)(a.x[c2] + xr * d + q * 4) = vals[k];
      }
    }
    ln_row4<RQ>(vals, d, a.g[c2], a.b[c2], a.a[c2] + xr * d, red);
  }
}

// k_rows with the fewest float4 groups a thread that cover a row of d
void launch_rows(const RowsArgs& r, int rows, hipStream_t st) {
  const int nq = r.d / 4;
  if (nq <= ROWT) hipLaunchKernelGGL(k_rows<1>, dim3(rows), dim3(ROWT), 0, st, r);
  else if (nq <= 2 * ROWT) hipLaunchKernelGGL(k_rows<2>, dim3(rows), dim3(ROWT), 0, st, r);
  else hipLaunchKernelGGL(k_rows<ROWQ>, dim3(rows), dim3(ROWT), 0, st, r);
}

// XATT: the cross attention of one block pass from the per-draft factors A_h = Wq_h^T K_h^T and
// B_h = Wo_h V_h (both [H][C][d] fp16) and sb_h[c] = bq_h . K_h[c] (fp32): for every row r,
//   scores[r][c] = (LN(x)[r] . A_h[c] + sb_h[c]) / sqrt(hd),  P = softmax_c(scores),
//   out_h[r][n] = sum_c P[r][c] B_h[c][n]
// (exactly q_h . K_h with q = Wq LN(x) + bq, and Wo_h (P V_h); A and B are rounded to fp16 where
// the reference rounds q and P V_h).  One workgroup per (expert, head, column block of n), one
// column of the block per thread.  The workgroup first puts its columns of B_h in flight (they do
// not depend on the scores), then the scores: one 16 x 16 MFMA tile (rows x context rows) over d
// with the k-steps split over the waves, each wave issuing all its loads before its MFMAs, the wave
// tiles summed through LDS; the softmax, 16 lanes a row; and its columns of P_h B_h, written as the
// head's fp32 partial [H][S][d] that the residual row kernel sums with the other heads and the
// out_proj bias, as for any split-K sublayer.  LN(x) and each A_h arrive as MFMA operand images
// (frag_index order): the score phase is bound by what one CU pulls in, and a k-step's loads then
// read 4 S (4 C) contiguous vectors instead of 64-byte pieces of rows a row apart (measured:
// -2.8 us a launch at S = C = 8, d = 5120).
struct XattArgs {
  const h16* xn[4];      // LN_cross(x) rows [S][d], frag_index order
  const h16* A[4];       // this layer's A [H][C][d], each head's [C][d] in frag_index order
  const h16* Bf[4];      // this layer's B [H][C][d]
  const float* sb[4];    // this layer's sb [H][C]
  float* out[4];         // partials [H][S][d]
  int S[4];
  int Sr[4];             // rows per request (the S rows hold S / Sr requests)
  int Ssg[4];            // rows per subgroup (0: S): workgroups take the rows in subgroups of at
                         // most 16, each with its own requests' context rows
  int Ce[4];             // context rows of the entry's group (0: C)
  int nex, d, H, C, nb;  // C: context rows of all the group's requests (the most of any entry)
  int Cq;                // context rows per request: row r scores only its request's rows
  int nsg, Csg;          // subgroups, context rows per subgroup (0: C)
  float scale;
};

constexpr int XT = 512;        // threads of an XATT workgroup

template <int CM>              // context rows, padded to 8 or 16
__global__ void __launch_bounds__(XT) k_xattn(XattArgs a) {
  constexpr int NW = XT / 64;
  constexpr int XRS = CM == 8 ? 20 : 10;     // k-steps a wave loads in one round (registers)
  __shared__ float red[NW][256];
  __shared__ float P[MAXR][16];
  int b = blockIdx.x;
  const int cb = b % a.nb;
  b /= a.nb;
  const int sg = b % a.nsg;
  b /= a.nsg;
  const int h = b % a.H, e = b / a.H;
  // this subgroup's rows [r0, r0 + S) of the expert's St rows and context rows [c0, c0 + C) of Ct
  const int St = a.S[e], Ct = a.Ce[e] > 0 ? a.Ce[e] : a.C, d = a.d;
  const int Ssg = a.Ssg[e] > 0 ? a.Ssg[e] : St, Csg = a.Csg > 0 ? a.Csg : Ct;
  const int r0 = sg * Ssg, c0 = sg * Csg;
  const int S = min(Ssg, St - r0), C = min(Csg, Ct - c0);
  if (S <= 0 || C <= 0) return;                      // (a subgroup past the group's requests)
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // this thread's first column of B_h (every context row of the subgroup), in flight before the
  // scores; a block of more than XT columns gives the thread further columns XT apart
  const int cpb = d / a.nb, n = cb * cpb + min(t, cpb - 1);
  const h16* Bbase = a.Bf[e] + ((size_t)h * Ct + c0) * d;
  h16 bv[CM];
#pragma unroll
  for (int c = 0; c < CM; ++c) bv[c] = Bbase[(size_t)min(c, C - 1) * d + n];
  // scores: lane row = lane % 16, context row = lane % 16 of the B operand, k-group lane / 16.
  // Lanes of rows past S or context rows past C load nothing (zero operands).  The operand
  // images hold every row of the expert (St) and every context row (Ct).
  const h16* Ah = a.A[e] + (size_t)h * Ct * d;
  const int ns = d / 32, per = (ns + NW - 1) / NW, s0 = wave * per, s1 = min(ns, s0 + per);
  const int ci = lane & 15, kg = lane >> 4;
  const bool xl = ci < S, al = ci < C;
  const h16* xrow = a.xn[e] + ((size_t)kg * St + r0 + min(ci, S - 1)) * 8;    // + k-step * 4 St vectors
  const h16* arow = Ah + ((size_t)kg * Ct + c0 + min(ci, C - 1)) * 8;
  const h16x8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int r0 = s0; r0 < s1; r0 += XRS) {
    h16x8 xv[XRS], av[XRS];
#pragma unroll
    for (int u = 0; u < XRS; ++u) {
      const int st = min(r0 + u, s1 - 1);
      xv[u] = zero8;
      av[u] = zero8;
      if (xl) xv[u] = *(const h16x8*)(xrow + (size_t)st * 32 * St);
      if (al) av[u] = *(const h16x8*)(arow + (size_t)st * 32 * Ct);
    }
#pragma unroll
    for (int u = 0; u < XRS; ++u)
      if (r0 + u < s1) acc = mfma_f16(xv[u], av[u], acc);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) red[wave][(4 * (lane >> 4) + q) * 16 + (lane & 15)] = acc[q];
  __syncthreads();
  // the score of (row r, context row c) in thread 16 r + c; the softmax over the row's 16 lanes
  // (every row r < S has its own request's context rows)
  if (t < 256) {
    const int r = t >> 4, c = t & 15;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) v += red[w][t];
    const bool ok = r < S && c < C && c / a.Cq == r / a.Sr[e];
    const float sc = ok ? (v + a.sb[e][h * Ct + c0 + c]) * a.scale : -INFINITY;
    float m = sc;
    m = fmaxf(m, dpp_f32<DPP_XOR1>(m));
    m = fmaxf(m, dpp_f32<DPP_XOR2>(m));
    m = fmaxf(m, dpp_f32<DPP_HMIRROR>(m));
    m = fmaxf(m, dpp_f32<DPP_MIRROR>(m));
    const float z = ok ? expf(sc - m) : 0.f;
    const float sum = row_sum(z);
    if (r < S) P[r][c] = z * (1.0f / sum);     // 0 for masked and padding context rows
  }
  __syncthreads();
  // this thread's columns of P_h B_h
  for (int cc = t; cc < cpb; cc += XT) {
    const int nn = cb * cpb + cc;
    float* oh = a.out[e] + ((size_t)h * St + r0) * d + nn;
    float bf[CM];
    if (cc == t) {
#pragma unroll
      for (int c = 0; c < CM; ++c) bf[c] = (float)bv[c];
    } else {
#pragma unroll
      for (int c = 0; c < CM; ++c) bf[c] = (float)Bbase[(size_t)min(c, C - 1) * d + nn];
    }
    for (int r = 0; r < S; ++r) {
      float o = 0.f;
#pragma unroll
      for (int c = 0; c < CM; ++c) o += P[r][c] * bf[c];
      oh[(size_t)r * d] = o;
    }
  }
}

// The two-heads fold's operand rows: for every expert, block l and part (context K, then V), rows
// [j][c] = row c of the part with the columns of all but the j-th head of each 2 hd-wide k-chunk set
// to zero, so that one k-chunk's 2 C rows give both of its heads' factors apart.
struct FoldMaskArgs {
  const h16* kv[4];      // [L][2][C][d] (the cross K/V rows)
  h16* out[4];           // [L][2][2][C][d]
  int nex, nl, C, d, hd;
};

// (workgroup b of nb taking every nb-th run of blockDim vectors)
__device__ void fold_mask_rows(const FoldMaskArgs& a, int b, int nb) {
  const int nv = a.d / 8;                                        // 8-column vectors a row
  const size_t per_ex = (size_t)a.nl * 2 * 2 * a.C * nv;
  const size_t total = per_ex * a.nex;
  for (size_t i = (size_t)b * blockDim.x + threadIdx.x; i < total; i += (size_t)nb * blockDim.x) {
    const int e = (int)(i / per_ex);
    size_t t = i - (size_t)e * per_ex;
    const int v = (int)(t % nv);
    t /= nv;
    const int c = (int)(t % a.C);
    t /= a.C;
    const int j = (int)(t % 2);
    const size_t lp = t / 2;                                     // l * 2 + part
    const int col = v * 8;                                       // a vector lies inside one head
    const bool keep = ((col % (2 * a.hd)) >= a.hd) == (j == 1);
    const h16x8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
    const h16x8 x = *(const h16x8*)(a.kv[e] + (lp * a.C + c) * a.d + col);
    *(h16x8*)(a.out[e] + ((lp * 2 + j) * a.C + c) * a.d + col) = keep ? x : zero;
  }
}

// The query bias's share of every block's scores, sb[l][h][c] = bq_h . K_h[c], once per draft:
// one workgroup per (expert, block), one wave per (head, context row) pair at a time.
struct XbiasArgs {
  const h16* K[4];       // block 0's context K rows [C][d]; block l at + l * kstride halves
  const h16* bq[4];      // block 0's cross_attn.in_proj_bias[0:d]; block l at + l * bstride bytes
  float* sb[4];          // [L][H][C]
  long long kstride, bstride;
  int nex, nl, d, H, C;
  FoldMaskArgs fm;       // two-heads fold: its masked operand rows, by mask_wgs more workgroups
  int mask_wgs;
};

__global__ void __launch_bounds__(1024) k_xbias(XbiasArgs a) {
  if ((int)blockIdx.x >= a.nex * a.nl) {   // (independent of the scores: the same launch)
    fold_mask_rows(a.fm, blockIdx.x - a.nex * a.nl, a.mask_wgs);
    return;
  }
  const int e = blockIdx.x / a.nl, l = blockIdx.x - e * a.nl;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int hd = a.d / a.H;
  const h16* K = a.K[e] + (size_t)l * a.kstride;
  const h16* bq = (const h16*)((const char*)a.bq[e] + (size_t)l * a.bstride);
  // (the pairs of a wide group's many context rows spread over gridDim.y workgroups)
  for (int p = blockIdx.y * nw + wave; p < a.H * a.C; p += gridDim.y * nw) {
    const int h = p / a.C, c = p - h * a.C;
    float s = 0.f;
    for (int j = lane; j < hd; j += 64) s += (float)bq[h * hd + j] * (float)K[(size_t)c * a.d + h * hd + j];
    s = wave_sum(s);
    if (lane == 0) a.sb[e][((size_t)l * a.H + h) * a.C + c] = s;
  }
}

// Column blocks per (expert, head) of XATT: the fewest that give each thread at most one column
// (each block recomputes the head's scores, so more blocks only repeat that work); 0 if d has no
// such split.
// cols: the most columns a thread may take (each block recomputes its head's scores: the wide
// groups' many subgroups already fill the chip, so there a thread takes several columns).
int xattn_blocks(int d, int units, int cols = 1) {
  (void)units;
  for (int nb = 1; nb <= d; ++nb)
    if (d % nb == 0 && d / nb <= XT * cols && (d / nb <= XT || (d / nb) % XT == 0)) return nb;
  return 0;
}

int launch_xattn(const XattArgs& a, hipStream_t st) {
  const int Csg = a.Csg > 0 ? a.Csg : a.C;
  if (Csg > 16 || a.nb <= 0 || a.nsg < 1 || (long long)a.nsg * Csg < a.C) return CFH_E_UNSUPPORTED;
  for (int e = 0; e < a.nex; ++e) {
    const int Ssg = a.Ssg[e] > 0 ? a.Ssg[e] : a.S[e];
    if (Ssg > MAXR || (long long)a.nsg * Ssg < a.S[e]) return CFH_E_UNSUPPORTED;
  }
  const dim3 grid((unsigned)(a.nex * a.H * a.nsg * a.nb));
  if (Csg <= 8) hipLaunchKernelGGL(k_xattn<8>, grid, dim3(XT), 0, st, a);
  else hipLaunchKernelGGL(k_xattn<16>, grid, dim3(XT), 0, st, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// XBLK: the residual row after the self attention, the folded cross attention and the residual row
// after it, for one expert's S <= 8 rows in ONE workgroup, in place of RES -> XATT -> RES (one-request
// flows of width d <= 640, where those three launches cost ~17 us a block pass whatever they move):
//   x1 = x + (sum_kc P[kc] + b_o);  xn = fp16(LN_cross(fp16(x1)))
//   scores_h[r][c] = (xn[r] . A_h[c] + sb_h[c]) / sqrt(hd),  P_h = softmax_c
//   x2 = x1 + (sum_h sum_c P_h[r][c] B_h[c][n] + b_oc);  x <- x2;  a = fp16(LN_ffn(fp16(x2)))
// (fp16 residual mode: each add rounded as in RES).  The same operations as those kernels; the sums
// over d (LayerNorm statistics, scores) and over the heads' outputs run in another order, all in
// fp32.  The workgroup is one chain of dependent steps, so every load that does not depend on it --
// the partial rows, the residual row, both LayerNorms' weights, this wave's A and B fragments -- is
// issued first, and each phase then reads registers and LDS only.  Phases: a wave a row (x1,
// LN_cross into LDS); the scores of two heads as one 16 x 16 MFMA tile (rows x both heads' C <= 8
// context rows), k-steps split over two waves; the softmax, 8 lanes a (head, row); the heads'
// outputs as 16-column MFMA tiles over k = (head, context row); a wave a row (LN_ffn).
// Every load is unconditional, from a clamped address, the value selected afterwards: a load under
// a branch is waited for before the branch joins.
struct XbEx {
  float* x;               // residual rows [S][d], x -> x2 in place
  const float* P;         // self-attention out_proj partials [ks][S][d]
  h16* a;                 // out: LN_ffn rows [S][d]
  const h16* bo;          // self_attn.out_proj.bias
  const h16* gx;          // cross_norm weight / bias
  const h16* bx;
  const h16* A;           // this layer's A [H][C][d], each head's [C][d] in frag_index order
  const h16* Bf;          // this layer's B [H][C][d]
  const float* sb;        // this layer's sb [H][C]
  const h16* boc;         // cross_attn.out_proj.bias
  const h16* gf;          // ffn LayerNorm weight / bias
  const h16* bf;
  int S;
};

struct XblkArgs {
  XbEx ex[4];
  int nex, d, H, C, ks, mode;
  float scale;
};

constexpr int XBT = 512;        // threads of an XBLK workgroup: 8 waves, 256 VGPRs a lane
constexpr int XBR = XBT / 64;   // most rows (a wave a row)
constexpr int XBH = 8;          // most heads
constexpr int XBC = 8;          // most context rows (two heads' scores share a 16-column tile)

size_t xblock_lds(int S, int d, int H) {
  return (size_t)S * d * 4 + (size_t)S * (d + 8) * 2 + (size_t)XBR * 256 * 4 + (size_t)H * XBR * XBC * 4;
}

template <int MODE>   // RES_ADD32 or RES_ADD16
__device__ __forceinline__ float xb_upd(float x, float s, float b) {
  return MODE == RES_ADD16 ? r16(x + r16(s + b)) : x + (s + b);
}

__device__ __forceinline__ float h_lo(unsigned u) { return (float)__builtin_bit_cast(h16, (unsigned short)(u & 0xFFFFu)); }
__device__ __forceinline__ float h_hi(unsigned u) { return (float)__builtin_bit_cast(h16, (unsigned short)(u >> 16)); }

// LN of the fp16-rounded row v (NQJ float4 groups a lane, q = lane + 64 j) into out[0 .. d)
template <int NQJ>
__device__ __forceinline__ void xb_ln(float4 (&v)[NQJ], int d, const h16x4 (&g)[NQJ], const h16x4 (&b)[NQJ], h16* out) {
  const int lane = threadIdx.x & 63, nq = d / 4;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NQJ; ++j) {
    v[j] = lane + 64 * j < nq ? r16x4(v[j]) : make_float4(0.f, 0.f, 0.f, 0.f);
    s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  }
  const float mean = wave_sum(s) / (float)d;
  float q2 = 0.f;
#pragma unroll
  for (int j = 0; j < NQJ; ++j) {
    const float a0 = v[j].x - mean, a1 = v[j].y - mean, a2 = v[j].z - mean, a3 = v[j].w - mean;
    if (lane + 64 * j < nq) q2 += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
  }
  const float rstd = 1.0f / sqrtf(wave_sum(q2) / (float)d + LN_EPS);
#pragma unroll
  for (int j = 0; j < NQJ; ++j) {
    const int q = lane + 64 * j;
    h16x4 o;
    o[0] = (h16)((v[j].x - mean) * rstd * (float)g[j][0] + (float)b[j][0]);
    o[1] = (h16)((v[j].y - mean) * rstd * (float)g[j][1] + (float)b[j][1]);
    o[2] = (h16)((v[j].z - mean) * rstd * (float)g[j][2] + (float)b[j][2]);
    o[3] = (h16)((v[j].w - mean) * rstd * (float)g[j][3] + (float)b[j][3]);
    if (q < nq) *(h16x4*)(out + q * 4) = o;
  }
}

// MODE: residual update; NQJ: float4 groups a lane in a row (d <= 256 NQJ); KP: partial rows
// loaded up front (ks <= KP); TPW >= d / 128: column tiles of B a wave holds (and 2 TPW >= d / 64
// k-steps of A, half of d).
template <int MODE, int NQJ, int KP, int TPW>
__global__ void __launch_bounds__(XBT) k_xblock(XblkArgs a) {
  extern __shared__ __align__(16) float xl[];
  constexpr int XBA = 2 * TPW;
  const XbEx& ex = a.ex[blockIdx.x];
  const int S = ex.S, d = a.d, H = a.H, C = a.C, ks = a.ks, nq = d / 4, ldn = d + 8;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  float* x1 = xl;                                   // [S][d]: x1, then x2
  h16* xn = (h16*)(x1 + (size_t)S * d);             // [S][ldn]
  float* red = (float*)(xn + (size_t)S * ldn);      // [XBR][256] score tiles
  float* Pp = red + XBR * 256;                      // [H][XBR][XBC] probabilities
  const size_t Sd = (size_t)S * d;
  // ---- loads first.  Row phases: this wave's row (clamped), its partials, residual and weights
  const int rw = min(wave, S - 1);
  float4 pv[KP][NQJ], xo[NQJ];
  h16x4 bo[NQJ], gx[NQJ], bx[NQJ], gf[NQJ], bf[NQJ];
#pragma unroll
  for (int j = 0; j < NQJ; ++j) {
    const int q = min(lane + 64 * j, nq - 1);
#pragma unroll
    for (int u = 0; u < KP; ++u) pv[u][j] = *(const float4*)(ex.P + min(u, ks - 1) * Sd + (size_t)rw * d + q * 4);
    xo[j] = *(const float4*)(ex.x + (size_t)rw * d + q * 4);
    bo[j] = *(const h16x4*)(ex.bo + q * 4);
    gx[j] = *(const h16x4*)(ex.gx + q * 4);
    bx[j] = *(const h16x4*)(ex.bx + q * 4);
    gf[j] = *(const h16x4*)(ex.gf + q * 4);
    bf[j] = *(const h16x4*)(ex.bf + q * 4);
  }
  // scores: wave = pair + 4 kgrp takes heads 2 pair, 2 pair + 1 (tile columns ci < 8, >= 8) over
  // k-steps [kgrp half, ...); lanes of context rows past C or heads past H load clamped rows, whose
  // scores are masked
  const int ns = d / 32, half = (ns + 1) / 2, pair = wave & 3, st0 = (wave >> 2) * half;
  const int ci = lane & 15, kg = lane >> 4;
  const int hh = min(2 * pair + (ci >> 3), H - 1), cc = min(ci & 7, C - 1);
  const h16* arow = ex.A + (size_t)hh * C * d + ((size_t)kg * C + cc) * 8;
  const h16x8 zero8 = {0, 0, 0, 0, 0, 0, 0, 0};
  h16x8 av[XBA];
#pragma unroll
  for (int u = 0; u < XBA; ++u) av[u] = *(const h16x8*)(arow + (size_t)min(st0 + u, ns - 1) * 32 * C);
  // the softmax thread's score bias: head t >> 6, row (t >> 3) & 7, context row t & 7
  const float sbv = ex.sb[min(t >> 6, H - 1) * C + min(t & 7, C - 1)];
  // the heads' outputs as MFMA tiles (rows x 16 columns, k = 8 h + c over four heads a k-step): this
  // wave's column tiles T = wave + 8 u; lane (n, kg) holds B[h][c][16 T + n] for head h = 4 kc + kg,
  // c = 0 .. 7 (rows past C and heads past H clamped; their probabilities are zero)
  const int ntile = d / 16;
  h16x8 bfr[TPW][2];
  h16 bocv[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int n = 16 * min(wave + 8 * u, ntile - 1) + ci;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const h16* bp = ex.Bf + (size_t)min(4 * kc + kg, H - 1) * C * d + n;
#pragma unroll
      for (int c = 0; c < 8; ++c) bfr[u][kc][c] = bp[(size_t)min(c, C - 1) * d];
    }
    bocv[u] = ex.boc[n];
  }
  // ---- x1 = x + (sum of the partials in order + b_o); LN_cross -> xn
  if (wave < S) {
    float4 v[NQJ];
#pragma unroll
    for (int j = 0; j < NQJ; ++j) {
      v[j] = pv[0][j];
#pragma unroll
      for (int u = 1; u < KP; ++u)
        if (u < ks) { v[j].x += pv[u][j].x; v[j].y += pv[u][j].y; v[j].z += pv[u][j].z; v[j].w += pv[u][j].w; }
      float4 y;
      y.x = xb_upd<MODE>(xo[j].x, v[j].x, (float)bo[j][0]);
      y.y = xb_upd<MODE>(xo[j].y, v[j].y, (float)bo[j][1]);
      y.z = xb_upd<MODE>(xo[j].z, v[j].z, (float)bo[j][2]);
      y.w = xb_upd<MODE>(xo[j].w, v[j].w, (float)bo[j][3]);
      const int q = lane + 64 * j;
      if (q < nq) *(float4*)(x1 + (size_t)wave * d + q * 4) = y;
      v[j] = y;
    }
    xb_ln<NQJ>(v, d, gx, bx, xn + (size_t)wave * ldn);
  }
  __syncthreads();
  // ---- score tiles (A operand: xn rows, rows past S read row 0 and are never used)
  if (2 * pair < H) {
    const h16* xrow = xn + (size_t)(ci < S ? ci : 0) * ldn + kg * 8;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < XBA; ++u) {
      const int st = st0 + u;
      const bool in = u < half && st < ns;
      acc = mfma_f16(*(const h16x8*)(xrow + min(st, ns - 1) * 32), in ? av[u] : zero8, acc);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) red[wave * 256 + (4 * kg + q) * 16 + ci] = acc[q];
  }
  __syncthreads();
  // ---- softmax over the context rows, 8 lanes a (head, row)
  {
    const int h = t >> 6, r = (t >> 3) & 7, c = t & 7, pr = h >> 1, n = (h & 1) * 8 + c;
    if (h < H) {
      const float v = red[pr * 256 + r * 16 + n] + red[(pr + 4) * 256 + r * 16 + n];
      const bool ok = r < S && c < C;
      const float sc = ok ? (v + sbv) * a.scale : -INFINITY;
      float m = sc;
      m = fmaxf(m, dpp_f32<DPP_XOR1>(m));
      m = fmaxf(m, dpp_f32<DPP_XOR2>(m));
      m = fmaxf(m, dpp_f32<DPP_HMIRROR>(m));
      const float z = ok ? expf(sc - m) : 0.f;
      float sum = z;
      sum += dpp_f32<DPP_XOR1>(sum);
      sum += dpp_f32<DPP_XOR2>(sum);
      sum += dpp_f32<DPP_HMIRROR>(sum);
      Pp[(h * XBR + r) * XBC + c] = ok ? z * (1.0f / sum) : 0.f;
    }
  }
  __syncthreads();
  // ---- x2 = x1 + (sum_h P_h B_h + b_oc) as MFMA tiles.  The probabilities enter as fp16 pairs
  // p = hi + lo (hi = fp16(p), lo = fp16(p - hi)), so the products keep ~22 bits of p and every sum
  // is in fp32 (the sums over the context rows and heads in the MFMA's order)
  {
    const int r = ci;
    h16x8 ph[2], pl[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      const int h = 4 * kc + kg;
      const bool in = h < H && r < XBR;
      const float* pp = Pp + (min(h, H - 1) * XBR + min(r, XBR - 1)) * XBC;
      const float4 p0 = *(const float4*)pp, p1 = *(const float4*)(pp + 4);
      const float pc[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float v = in ? pc[c] : 0.f;
        ph[kc][c] = (h16)v;
        pl[kc][c] = (h16)(v - (float)ph[kc][c]);
      }
    }
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const int T = wave + 8 * u;
      if (T >= ntile) break;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        if (4 * kc >= H) break;
        acc = mfma_f16(ph[kc], bfr[u][kc], acc);
        acc = mfma_f16(pl[kc], bfr[u][kc], acc);
      }
      const int n = 16 * T + ci;
      const float b = (float)bocv[u];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = 4 * kg + q;
        if (i < S) {
          const float y = xb_upd<MODE>(x1[(size_t)i * d + n], acc[q], b);
          x1[(size_t)i * d + n] = y;
          ex.x[(size_t)i * d + n] = y;
        }
      }
    }
  }
  __syncthreads();
  // ---- LN_ffn of x2, a wave a row
  if (wave < S) {
    float4 v[NQJ];
#pragma unroll
    for (int j = 0; j < NQJ; ++j) v[j] = *(const float4*)(x1 + (size_t)wave * d + min(lane + 64 * j, nq - 1) * 4);
    xb_ln<NQJ>(v, d, gf, bf, ex.a + (size_t)wave * d);
  }
}

template <int MODE>
void launch_xblock_m(const XblkArgs& a, size_t lds, hipStream_t st) {
  const dim3 g(a.nex), b(XBT);
  if (a.d <= 512) {
    if (a.ks <= 4) hipLaunchKernelGGL((k_xblock<MODE, 2, 4, 4>), g, b, lds, st, a);
    else hipLaunchKernelGGL((k_xblock<MODE, 2, 8, 4>), g, b, lds, st, a);
  } else {
    hipLaunchKernelGGL((k_xblock<MODE, 3, 4, 5>), g, b, lds, st, a);   // (eight partial rows there spill)
  }
}

int launch_xblock(const XblkArgs& a, hipStream_t st) {
  int smax = 0;
  for (int e = 0; e < a.nex; ++e) smax = std::max(smax, a.ex[e].S);
  if (a.nex < 1 || a.nex > 4 || smax < 1 || smax > XBR || a.d > 640 || a.d % 32 || a.C < 1 || a.C > XBC ||
      a.H < 1 || a.H > XBH || a.ks < 1 || a.ks > (a.d <= 512 ? 8 : 4) || (a.mode != RES_ADD32 && a.mode != RES_ADD16))
    return CFH_E_UNSUPPORTED;
  const size_t lds = xblock_lds(smax, a.d, a.H);
  if (lds > 64 * 1024) return CFH_E_UNSUPPORTED;
  if (a.mode == RES_ADD16) launch_xblock_m<RES_ADD16>(a, lds, st);
  else launch_xblock_m<RES_ADD32>(a, lds, st);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

// Launch shapes of the wide kernels with `groups` request groups a launch.
struct WideShape {
  int groups;
  int wv_qkv, wv_w1, wv_kv, wv_qc; // full-K launches: waves per workgroup (wv_qc: unfolded cross q)
  int wv_split;                    // split-K launches: waves per workgroup
  int ks_wo, ks_ww2, ks_wout, ks_oc;  //                and k-splits (ks_oc: unfolded cross out-proj)
  bool ok;
};

struct Plan {
  int d, fd, CS, E, NL, C, KD, H, hd, nch, Smax;
  int R, Ct;          // requests per group (rows packed in one tile) and their context rows R C
  int ks_att;         // k-chunks of the attention launches: H / heads per chunk
  int ks_qc, ks_w2, ks_out, ks_kv;
  int wpb_qc, wpb_w2, wpb_out, tpw_att, wpb_att, wpb_full, wpb_w1;
  int pks;            // partial slots per expert
  int res_mode;       // RES_ADD32 (fused-kernel numerics) or RES_ADD16 (torch fp16 modules)
  bool fold;          // cross attention folded into per-draft factors (cfh::xattn_fold / xattn_fold2)
  bool fold2;         // ... built two heads a k-chunk from operand rows masked per head (xattn_fold2)
  int ks_fold, S_fold; // the factor launch's k-chunks and operand rows
  bool conc;          // chunk experts on concurrent streams within an Euler step (conc_experts)
  int wpb_fold, xnb;  // fold hoist launch waves / XATT column blocks per (expert, head)
  bool xblk;          // one request, folded, d <= 640: residual, cross attention and residual
                      // rows in one XBLK launch (k_xblock) instead of three
  bool wide;          // more than two requests a group: every row of the group shares each weight
                      // stream through the chunked-staging kernels (cfh_wide.h)
  WideShape ws[2];    // wide launch shapes for one group a launch, and for two (ws[1].ok: a batch of
                      // several groups runs two at a time, both groups' entries in every launch)
  bool ok;
};

// Waves per workgroup of a wide launch whose workgroups should all be resident at once: the most
// workgroups up to one per CU, then the most waves.  Two request groups of one expert then stream
// each weight fragment side by side (on one XCD, `WArgs::pair`), and the second read hits the L2:
// W1 at d = 4096 for two 16-request groups took 96.7 us a launch as 256 workgroups of 12 waves
// (one group alone: 79.5 us), 127-135 us as 512 of 6 or 768 of 4, 159 us when the groups' reads
// did not coincide.
int wide_wv_resident(int tiles, int units) {
  constexpr int CUS = 256;
  int best = 0;
  long long best_wgs = 0;
  for (int wv : {4, 6, 8, 12}) {
    if (tiles % (WT * wv)) continue;
    const long long wgs = (long long)units * tiles / (WT * wv);
    if (wgs > CUS) continue;
    if (!best || wgs > best_wgs || (wgs == best_wgs && wv > best)) {
      best = wv;
      best_wgs = wgs;
    }
  }
  return best ? best : wide_wv(tiles, units);
}

// Wide launch shapes for `groups` request groups a launch: about one workgroup per CU for each
// streaming launch (every chunk expert of every group in one launch).
WideShape wide_shape(const Plan& p, int groups) {
  WideShape s = {};
  s.groups = groups;
  const int units = groups * p.nch;
  if (units > 4) return s;
  constexpr int CUS = 256;
  // split-K launches: 4-wave workgroups for one group; for two, 8-wave ones at one workgroup per CU,
  // so that the two groups' workgroups of a unit run together (d = 4096, 16 + 16 requests, E = 2:
  // 8.34 against 8.90 ms a flow pass with 4-wave workgroups)
  s.wv_split = groups > 1 && (p.d / 16) % (WT * 8) == 0 ? 8 : 4;
  auto ks_split = [&](int N, int K) {
    int best = 0;
    for (int ks = 1; ks <= K / WCH; ++ks) {
      if (K % ks || (K / ks) % WCH) continue;
      best = ks;
      if ((long long)units * (N / 16 / (WT * s.wv_split)) * ks >= CUS) break;
    }
    return best;
  };
  auto wv_full = [&](int N) { return groups > 1 ? wide_wv_resident(N / 16, units) : wide_wv(N / 16, units); };
  s.wv_qkv = wv_full(3 * p.d);
  s.wv_w1 = wv_full(p.fd);
  s.wv_kv = wide_wv(2 * p.d / 16, std::min(4, groups * std::min(4 / groups, p.nch * p.NL)));
  s.ks_wo = ks_split(p.d, p.d);
  s.ks_ww2 = ks_split(p.d, p.fd);
  s.ks_wout = ks_split(p.d, p.d);
  s.wv_qc = p.fold ? 0 : wv_full(p.d);
  s.ks_oc = p.fold ? 0 : ks_split(p.d, p.d);
  auto wa = [&](int N, int K, int ks, int nex) {
    WArgs a = {};
    a.nex = nex; a.N = N; a.K = K; a.ks = ks; a.pair = groups > 1;
    return a;
  };
  const int kv_nex = groups * std::min(4 / groups, p.nch * p.NL);
  s.ok = s.ks_wo > 0 && s.ks_ww2 > 0 && s.ks_wout > 0 &&
         !wide_check(wa(3 * p.d, p.d, 1, units), s.wv_qkv, p.Smax) &&
         !wide_check(wa(p.fd, p.d, 1, units), s.wv_w1, p.Smax) &&
         !wide_check(wa(2 * p.d, p.d, 1, kv_nex), s.wv_kv, p.Ct) &&
         !wide_check(wa(p.d, p.d, s.ks_wo, units), s.wv_split, p.Smax) &&
         !wide_check(wa(p.d, p.fd, s.ks_ww2, units), s.wv_split, p.Smax) &&
         !wide_check(wa(p.d, p.d, s.ks_wout, units), s.wv_split, p.Smax) &&
         (p.fold ? !wide_check(wa(p.d, p.d, p.H, groups * p.nch), 4, p.Ct)
                 : s.ks_oc > 0 && !wide_check(wa(p.d, p.d, 1, units), s.wv_qc, p.Smax) &&
                       !wide_check(wa(p.d, p.d, s.ks_oc, units), s.wv_split, p.Smax));
  return s;
}

// Wide plan: both launch shapes, and whether every launch of the draft fits the wide kernels.
void make_wide_plan(Plan& p, const cfh_flow_dims* dm) {
  p.wide = true;
  p.conc = false;
  p.fold = cfh::xattn_fold(dm);
  p.fold2 = false;
  p.ks_fold = p.H;
  p.S_fold = p.Ct;
  // the cross attention folded (one head a k-chunk: its factors split-K by head need head widths
  // of whole staging chunks) or unfolded (q projection, attention per (request, head), out-proj)
  p.ok = (p.fold ? p.hd % WCH == 0 : p.hd % 8 == 0) && p.d % WCH == 0 && p.fd % WCH == 0 &&
         p.Smax <= WMAXR && p.Ct <= WMAXR && p.C <= 8 && 2 * p.KD <= MAXR && res_nq(p.d) > 0;
  if (!p.ok) return;
  p.ws[0] = wide_shape(p, 1);
  p.ws[1] = wide_shape(p, 2);
  p.pks = p.fold ? p.H : 1;
  for (const WideShape& w : p.ws)
    if (w.ok) p.pks = std::max({p.pks, w.ks_wo, w.ks_ww2, w.ks_wout, w.ks_oc});
  p.xnb = p.fold ? xattn_blocks(p.d, p.nch * p.H, 4) : 0;
  p.ok = p.ws[0].ok && (!p.fold || p.xnb > 0) &&
         (size_t)3 * p.KD * p.hd * 2 + (size_t)p.KD * p.KD * 4 <= 64 * 1024 &&   // self attention's LDS
         (p.fold || cross_attn_lds(p.KD, p.C, p.hd) <= 64 * 1024);
}

Plan make_plan(const cfh_flow_dims* dm, int R = 1) {
  Plan p = {};
  p.d = dm->d; p.fd = dm->ffn_mult * dm->d; p.CS = dm->chunk_size; p.E = dm->flow_steps;
  p.NL = dm->layers; p.C = dm->ctx_rows; p.KD = dm->draft_length; p.H = dm->heads; p.hd = p.d / p.H;
  p.ks_att = cfh::heads_per_chunk(p.hd, p.H) ? p.H / cfh::heads_per_chunk(p.hd, p.H) : 0;
  p.nch = p.KD / p.CS;
  p.R = R;
  p.Ct = R * p.C;
  p.Smax = R * p.KD;
  const int out_rows = R == 1 ? p.CS : p.Smax;   // OUT: the current chunk's rows, or every row when packed
  p.res_mode = dm->numerics == CFH_FLOW_MODULES ? RES_ADD16 : RES_ADD32;
  if (p.Smax > MAXR) {
    make_wide_plan(p, dm);
    return p;
  }
  p.fold = cfh::xattn_fold(dm);
  // two heads per k-chunk: folded for single-request groups only (2 x Ct operand rows per tile)
  p.fold2 = !p.fold && cfh::xattn_fold2(dm) && 2 * p.Ct <= 16;
  p.fold = p.fold || p.fold2;
  p.ks_fold = p.fold2 ? p.H / 2 : p.H;
  p.S_fold = p.fold2 ? 2 * p.Ct : p.Ct;
  // Concurrent chunk experts double the block passes' launches; below d = 1024 the host's launch
  // rate, not the GPU, then sets the pace of an eager draft (the latent flow at d = 640: +0.13 ms a
  // draft on two streams), so narrow shapes keep every expert in one launch.
  p.conc = p.nch > 1 && p.d >= 1024;
  const int tiles_d = p.d / 16;
  const size_t cap = 96 * 1024;
  // (one k-chunk when K has fewer than 8 k-steps: small latent widths)
  p.ks_qc = std::max(choose_ks(p.nch, tiles_d, p.d, p.Smax, 2048, cap), 1);
  // W2: one d-wide k-chunk per ffn slice (ks = ffn_mult) in 16-wave workgroups, so that W1 and W2
  // both run as one round of ~240 workgroups at one workgroup per CU; else split-K by wave count
  const bool w2_wide = tiles_d % 16 == 0 && stream_lds(S_BUF, p.Smax, p.d, p.hd, p.C) <= 150 * 1024;
  p.ks_w2 = w2_wide ? dm->ffn_mult : std::max(choose_ks(p.nch, tiles_d, p.fd, p.Smax, 4096, cap), 1);
  p.ks_out = std::max(choose_ks(p.nch, tiles_d, p.d, out_rows, 2048, cap), 1);
  p.ks_kv = ksplit_for(p.nch * p.NL, 2 * p.d / 16, p.d, p.Ct);
  p.wpb_w2 = w2_wide ? wpb_for_grid(tiles_d, p.nch * p.ks_w2, 16, p.Smax * (p.fd / p.ks_w2) / 8)
                     : std::min(4, pick_wpb(tiles_d, 1));
  p.wpb_out = wpb_for_grid(tiles_d, p.nch * p.ks_out, 8, out_rows * (p.d / p.ks_out) / 8);
  p.tpw_att = (tiles_d % 16 == 0) ? 2 : 1;
  p.wpb_att = pick_wpb(tiles_d, p.tpw_att);   // (the attention staging needs the waves' slots)
  fit_grid(tiles_d, p.nch * p.ks_att, &p.wpb_att, &p.tpw_att);
  // full-K launches (QKV, W1): one workgroup per CU at any width (16 waves for W1 and 8 for QKV
  // at d = 5120, fewer at narrow widths, where those would leave most CUs idle)
  p.wpb_full = wpb_for_grid(3 * tiles_d, p.nch, 8, p.Smax * p.d / 8);
  p.wpb_w1 = wpb_for_grid(p.fd / 16, p.nch, 16, p.Smax * p.d / 8);
  // the cross attention holds every q partial of its groups in registers: fewer QC splits if needed
  for (int ks = p.ks_qc; ks > 1; --ks) {
    SArgs a = {};
    a.N = p.d; a.K = p.d; a.ks = p.ks_att; a.wpb = p.wpb_att; a.tpw = p.tpw_att; a.hd = p.hd; a.ks_in = ks; a.Ck = p.Ct;
    if ((p.d / 32) % ks || stage_need(S_CROSS, a, p.Smax) > stage_slots(a.wpb)) continue;
    p.ks_qc = ks;
    break;
  }
  p.wpb_qc = wpb_for_grid(tiles_d, p.nch * p.ks_qc, 4, p.Smax * (p.d / p.ks_qc) / 8);
  fit_grid(tiles_d, p.nch * p.ks_qc, &p.wpb_qc, nullptr);
  fit_grid(tiles_d, p.nch * p.ks_out, &p.wpb_out, nullptr);
  p.pks = std::max(std::max(p.ks_att, p.ks_w2), p.ks_out);
  if (p.fold) p.pks = std::max(p.pks, p.H);   // the folded cross attention's per-head partials
  if (p.fold) {
    p.wpb_fold = wpb_for_grid(tiles_d, 2 * p.nch * p.ks_fold, 8, p.S_fold * (p.d / p.ks_fold) / 8);
    p.xnb = xattn_blocks(p.d, p.nch * p.H);
  }
  p.ok = p.ks_qc > 0 && p.ks_qc <= 8 && p.ks_w2 > 0 && p.ks_out > 0 && p.ks_att > 0 && res_nq(p.d) > 0 &&
         p.Smax <= MAXR && p.Ct <= 16;
  if (!p.ok) return p;
  // every streaming launch of a draft, as block_pass and the OUT step issue them
  auto sa = [&](int N, int K, int ks, int wpb, int tpw) {
    SArgs a = {};
    a.nex = p.nch; a.N = N; a.K = K; a.ks = ks; a.wpb = wpb; a.tpw = tpw; a.d = p.d; a.hd = p.hd;
    a.ks_in = p.ks_qc; a.Ck = p.Ct;
    return a;
  };
  auto unfolded_ok = [&]() {
    return !stream_check(S_BUF, sa(p.d, p.d, p.ks_qc, p.wpb_qc, 1), p.Smax) &&
           !stream_check(S_CROSS, sa(p.d, p.d, p.ks_att, p.wpb_att, p.tpw_att), p.Smax);
  };
  bool cross_ok = p.fold ? !stream_check(S_BUF, sa(p.d, p.d, p.ks_fold, p.wpb_fold, 1), p.S_fold) && p.xnb > 0
                         : unfolded_ok();
  if (!cross_ok && p.fold2) {
    // the two-heads fold does not fit this shape: the unfolded launches, with the partial slots they
    // need (a host-side scan of every supported shape -- d up to 16384, 1-128 heads, 4-16 context
    // rows, ffn 2/4/6, draft length 8/16 -- found none that takes this branch; it is kept so that a
    // shape the scan missed still runs)
    p.fold = p.fold2 = false;
    p.pks = std::max(std::max(p.ks_att, p.ks_w2), p.ks_out);
    p.ks_fold = p.S_fold = p.wpb_fold = p.xnb = 0;
    cross_ok = unfolded_ok();
  }
  p.ok = !stream_check(S_BUF, sa(3 * p.d, p.d, 1, p.wpb_full, 1), p.Smax) &&
         !stream_check(S_SELF, sa(p.d, p.d, p.ks_att, p.wpb_att, p.tpw_att), p.Smax) && cross_ok &&
         !stream_check(S_BUF, sa(p.fd, p.d, 1, p.wpb_w1, 1), p.Smax) &&
         !stream_check(S_BUF, sa(p.d, p.fd, p.ks_w2, p.wpb_w2, 1), p.Smax) &&
         !stream_check(S_BUF, sa(p.d, p.d, p.ks_out, p.wpb_out, 1), out_rows);
  p.xblk = p.ok && p.fold && R == 1 && p.d <= 640 && p.d % 32 == 0 && p.H <= XBH && p.Ct <= XBC &&
           p.Smax <= XBR && p.ks_att <= (p.d <= 512 ? 8 : 4) && xblock_lds(p.Smax, p.d, p.H) <= 64 * 1024;
  return p;
}

// Requests per group for a batch.  Wide groups (allow_wide, more than two requests): the batch in
// as few groups of at most WMAXR / draft_length requests as possible, balanced; otherwise the
// most requests (up to `batch`) whose rows fit one 16-row tile and whose plan this build runs.
// 1 always works when the shape is supported.
int group_size(const cfh_flow_dims* dm, int batch, bool allow_wide = true) {
  const int KD = dm->draft_length;
  if (allow_wide && batch * KD > MAXR && WMAXR / KD >= 3) {
    const int rmax = WMAXR / KD, ng = (batch + rmax - 1) / rmax, R = (batch + ng - 1) / ng;
    if (R * KD > MAXR && make_plan(dm, R).ok) return R;
  }
  for (int R = std::min(batch, MAXR / KD); R > 1; --R)
    if (make_plan(dm, R).ok) return R;
  return 1;
}

struct WS {
  float* z;
  float* x[4];
  h16* abuf[4];
  h16* qkv[4];
  h16* g[4];
  float* P[4];        // partials of the split-K kernels (O, OC, W2, OUT)
  float* Pq[4];       // cross-q partials (QC), read by OC (unfolded shapes)
  h16* kvc[4];        // [L][2][C][d]
  h16* fa[4];         // folded shapes: A [L][H][C][d] = Wq_h^T K_h^T
  h16* fb[4];         //                B [L][H][C][d] = Wo_h V_h
  float* fsb[4];      //                sb [L][H][C] = bq_h . K_h
  h16* fm[4];         // fold2: context K / V rows masked per head [L][2][2][C][d] (K/V, head in chunk)
  h16* cln[4];        // wide: context_norm(ctx) rows of every block [L][C][d]
  float* Pkv;         // [nch][L][ks][C][2d]
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
  w.z = (float*)take((size_t)p.R * p.KD * d * 4);
  for (int c = 0; c < p.nch; ++c) {
    const size_t S = (size_t)p.R * (c + 1) * p.CS;
    w.x[c] = (float*)take(S * d * 4);
    w.abuf[c] = (h16*)take(S * d * 2);
    w.qkv[c] = (h16*)take(S * 3 * d * 2);
    w.g[c] = (h16*)take(S * fd * 2);
    w.P[c] = (float*)take((size_t)p.pks * S * d * 4);
    if (!p.fold) w.Pq[c] = (float*)take((size_t)p.ks_qc * S * d * 4);
    w.kvc[c] = (h16*)take((size_t)p.NL * 2 * p.Ct * d * 2);
    if (p.fold) {
      w.fa[c] = (h16*)take((size_t)p.NL * p.H * p.Ct * d * 2);
      w.fb[c] = (h16*)take((size_t)p.NL * p.H * p.Ct * d * 2);
      w.fsb[c] = (float*)take((size_t)p.NL * p.H * p.Ct * 4);
    }
    if (p.fold2) w.fm[c] = (h16*)take((size_t)p.NL * 2 * 2 * p.Ct * d * 2);
    if (p.wide) w.cln[c] = (h16*)take((size_t)p.NL * p.Ct * d * 2);
  }
  if (!p.wide) w.Pkv = (float*)take((size_t)p.nch * p.NL * p.ks_kv * p.Ct * 2 * d * 4);
  w.ctx_mom = (float*)take((size_t)p.Ct * 2 * 4);
  w.total = off;
  return w;
}

// The workspace seen from chunk expert c0: its buffers at index 0.
WS expert_view(const WS& w, int c0) {
  WS v = w;
  for (int c = 0; c + c0 < 4; ++c) {
    v.x[c] = w.x[c + c0]; v.abuf[c] = w.abuf[c + c0]; v.qkv[c] = w.qkv[c + c0]; v.g[c] = w.g[c + c0];
    v.P[c] = w.P[c + c0]; v.Pq[c] = w.Pq[c + c0]; v.kvc[c] = w.kvc[c + c0];
    v.fa[c] = w.fa[c + c0]; v.fb[c] = w.fb[c + c0]; v.fsb[c] = w.fsb[c + c0]; v.fm[c] = w.fm[c + c0];
    v.cln[c] = w.cln[c + c0];
  }
  return v;
}

// Where a chunk expert's first block pass of a draft may start, relative to the previous expert's
// (concurrent experts): after that expert's STAGGER_AT-th launch of its first block (0: at once).
// After the fifth (the residual row before W1, ~100 us into a ~290 us block at d = 5120) one
// expert's row kernels and cross attention fall inside the other's W1 / W2 streams instead of
// beside its own: measured -0.2 ms a draft at d = 5120, no change at d = 2560 or 4096.
constexpr int STAGGER_AT = 5;

// The eight launches of block l (nine unfolded, six with XBLK) for chunk experts c0 .. c0 + nc - 1, every launch
// covering those experts; `mark`, if given, is recorded after the block's STAGGER_AT-th launch.
int block_pass(const Plan& p, const cfh::ExpertLayout& L, const WS& w_all, const void* const* experts_all,
               int l, int Rg, hipStream_t st, int c0, int nc, hipEvent_t mark = nullptr) {
  const WS w = expert_view(w_all, c0);
  const void* const* experts = experts_all + c0;
  const int d = p.d, fd = p.fd, NL = p.NL, nch = nc, Cg = Rg * p.C;
  auto PTR = [&](int c, size_t off) { return (const char*)experts[c] + off; };
  const size_t B = L.blk0 + (size_t)l * L.blkstride;
  auto S_of = [&](int c) { return Rg * (c0 + c + 1) * p.CS; };   // rows of expert c0 + c: Rg requests
  auto Sr_of = [&](int c) { return (c0 + c + 1) * p.CS; };       // rows per request
  int rc, launched = 0;
  const int stagger = p.xblk ? STAGGER_AT - 2 : STAGGER_AT;   // (XBLK: two launches fewer before W1)
  auto done = [&]() -> int {
    if (mark && ++launched == stagger) CFH_HIP(hipEventRecord(mark, st));
    return CFH_OK;
  };
  // QKV: q, k, v = fp16(LN_self(x) W_in^T + b_in), full-K tiles
  {
    SArgs a = {};
    a.conc = p.nch / nc;
    a.nex = nch; a.N = 3 * d; a.K = d; a.ks = 1; a.wpb = p.wpb_full; a.tpw = 1; a.d = d; a.hd = p.hd;
    a.wg_per_kc = (3 * d / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.qkv); x.a = w.abuf[c]; x.lda = d; x.bias = (const h16*)PTR(c, B + L.qkv_b);
      x.out = w.qkv[c]; x.S = S_of(c);
    }
    if ((rc = launch_stream<S_BUF, E_BIAS16>(a, p.Smax, st)) || (rc = done())) return rc;
  }
  // O: causal self attention per head, staged, then out_proj split-K by head (group)
  {
    SArgs a = {};
    a.conc = p.nch / nc;
    a.nex = nch; a.N = d; a.K = d; a.ks = p.ks_att; a.wpb = p.wpb_att; a.tpw = p.tpw_att; a.d = d; a.hd = p.hd;
    a.causal = 1;
    a.wg_per_kc = (d / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.o); x.a = w.qkv[c]; x.out = w.P[c]; x.S = S_of(c); x.Sr = Sr_of(c);
    }
    if ((rc = launch_stream<S_SELF, E_PART>(a, p.Smax, st)) || (rc = done())) return rc;
  }
  // XBLK: residual + LN_cross, the folded cross attention, residual + LN_ffn in one launch
  if (p.xblk) {
    XblkArgs x = {};
    x.nex = nch; x.d = d; x.H = p.H; x.C = Cg; x.ks = p.ks_att; x.mode = p.res_mode;
    x.scale = 1.0f / sqrtf((float)p.hd);
    const size_t per_l = (size_t)p.H * Cg * d;
    for (int c = 0; c < nch; ++c) {
      XbEx& e = x.ex[c];
      e.x = w.x[c]; e.P = w.P[c]; e.a = w.abuf[c]; e.S = S_of(c);
      e.bo = (const h16*)PTR(c, B + L.o_b);
      e.gx = (const h16*)PTR(c, B + L.xn_w); e.bx = (const h16*)PTR(c, B + L.xn_b);
      e.A = w.fa[c] + (size_t)l * per_l; e.Bf = w.fb[c] + (size_t)l * per_l;
      e.sb = w.fsb[c] + (size_t)l * p.H * Cg;
      e.boc = (const h16*)PTR(c, B + L.oc_b);
      e.gf = (const h16*)PTR(c, B + L.fn_w); e.bf = (const h16*)PTR(c, B + L.fn_b);
    }
    if ((rc = launch_xblock(x, st)) || (rc = done())) return rc;
  }
  ResArgs r = {};
  r.nex = nch; r.d = d; r.mode = p.res_mode;
  for (int c = 0; c < nch; ++c) { r.x[c] = w.x[c]; r.P[c] = w.P[c]; r.a[c] = w.abuf[c]; r.rows[c] = S_of(c); }
  // residual + LN_cross
  r.ks = p.ks_att;
  for (int c = 0; c < nch; ++c) {
    r.bias[c] = (const h16*)PTR(c, B + L.o_b);
    r.g[c] = (const h16*)PTR(c, B + L.xn_w); r.b[c] = (const h16*)PTR(c, B + L.xn_b);
  }
  r.pack = p.fold;   // the folded cross attention takes LN_cross(x) as an MFMA operand image
  if (!p.xblk && ((rc = launch_res(r, st)) || (rc = done()))) return rc;
  r.pack = 0;
  if (p.fold && !p.xblk) {
    XattArgs x = {};
    x.nex = nch; x.d = d; x.H = p.H; x.C = Cg; x.Cq = p.C; x.nb = p.xnb; x.scale = 1.0f / sqrtf((float)p.hd);
    x.nsg = 1;
    const size_t per_l = (size_t)p.H * Cg * d;
    for (int c = 0; c < nch; ++c) {
      x.xn[c] = w.abuf[c]; x.A[c] = w.fa[c] + (size_t)l * per_l; x.Bf[c] = w.fb[c] + (size_t)l * per_l;
      x.sb[c] = w.fsb[c] + (size_t)l * p.H * Cg;
      x.out[c] = w.P[c]; x.S[c] = S_of(c); x.Sr[c] = Sr_of(c);
    }
    if ((rc = launch_xattn(x, st)) || (rc = done())) return rc;
  }
  // QC: cross-attention query projection, split-K partials
  if (!p.fold) {
    SArgs a = {};
    a.conc = p.nch / nc;
    a.nex = nch; a.N = d; a.K = d; a.ks = p.ks_qc; a.wpb = p.wpb_qc; a.tpw = 1; a.d = d; a.hd = p.hd;
    a.wg_per_kc = (d / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.qc); x.a = w.abuf[c]; x.lda = d; x.out = w.Pq[c]; x.S = S_of(c);
    }
    if ((rc = launch_stream<S_BUF, E_PART>(a, p.Smax, st)) || (rc = done())) return rc;
  }
  // OC: cross attention per head over the hoisted context K/V, staged, then out_proj split-K by head
  if (!p.fold) {
    SArgs a = {};
    a.conc = p.nch / nc;
    a.nex = nch; a.N = d; a.K = d; a.ks = p.ks_att; a.wpb = p.wpb_att; a.tpw = p.tpw_att; a.d = d; a.hd = p.hd;
    a.ks_in = p.ks_qc; a.Ck = Cg; a.Cr = p.C;
    a.wg_per_kc = (d / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.oc); x.a = w.kvc[c] + (size_t)l * 2 * Cg * d; x.pin = w.Pq[c];
      x.bin = (const h16*)PTR(c, B + L.qc_b); x.out = w.P[c]; x.S = S_of(c); x.Sr = Sr_of(c);
    }
    if ((rc = launch_stream<S_CROSS, E_PART>(a, p.Smax, st)) || (rc = done())) return rc;
  }
  // residual + LN_ffn (the folded cross attention leaves one partial per head, OC one per k-chunk)
  r.ks = p.fold ? p.H : p.ks_att;
  for (int c = 0; c < nch; ++c) {
    r.bias[c] = (const h16*)PTR(c, B + L.oc_b);
    r.g[c] = (const h16*)PTR(c, B + L.fn_w); r.b[c] = (const h16*)PTR(c, B + L.fn_b);
  }
  if (!p.xblk && ((rc = launch_res(r, st)) || (rc = done()))) return rc;
  // W1: g = fp16(gelu(LN_ffn(x) W1^T + b1)), full-K tiles
  {
    SArgs a = {};
    a.conc = p.nch / nc;
    a.nex = nch; a.N = fd; a.K = d; a.ks = 1; a.wpb = p.wpb_w1; a.tpw = 1; a.d = d; a.hd = p.hd;
    a.gelu_r16 = p.res_mode == RES_ADD16;   // torch's Linear rounds before its GELU module
    a.wg_per_kc = (fd / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.w1); x.a = w.abuf[c]; x.lda = d; x.bias = (const h16*)PTR(c, B + L.w1_b);
      x.out = w.g[c]; x.S = S_of(c);
    }
    if ((rc = launch_stream<S_BUF, E_GELU16>(a, p.Smax, st)) || (rc = done())) return rc;
  }
  // W2: split-K partials
  {
    SArgs a = {};
    a.conc = p.nch / nc;
    a.nex = nch; a.N = d; a.K = fd; a.ks = p.ks_w2; a.wpb = p.wpb_w2; a.tpw = 1; a.d = d; a.hd = p.hd;
    a.wg_per_kc = (d / 16) / (a.wpb * a.tpw);
    for (int c = 0; c < nch; ++c) {
      SEx& x = a.ex[c];
      x.w = (const h16x8*)PTR(c, B + L.w2); x.a = w.g[c]; x.lda = fd; x.out = w.P[c]; x.S = S_of(c);
    }
    if ((rc = launch_stream<S_BUF, E_PART>(a, p.Smax, st)) || (rc = done())) return rc;
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
  if ((rc = launch_res(r, st))) return rc;
  return done();
}

// One request group of a wide launch sequence: its workspace, its requests [g0, g0 + Rg) of the
// batch and their context rows.
struct GroupRun {
  WS w;
  int g0, Rg;
  const h16* ctx;
};

// The launches of block l for `ng` request groups -- QKV, self attention, O, residual, folded cross
// attention (in subgroups of two requests), residual, W1, W2, residual; every chunk expert of every
// group in each launch (one group, or two whose entries share every launch:
// entry g * nch + c is expert c of group g, and `WArgs::pair` runs the two groups' workgroups of a
// weight unit side by side).
int block_pass_wide(const Plan& p, const WideShape& sh, const cfh::ExpertLayout& L, const GroupRun* gr, int ng,
                    const void* const* experts, int l, hipStream_t st) {
  const int d = p.d, fd = p.fd, NL = p.NL, nch = p.nch, nex = ng * nch;
  auto PTR = [&](int c, size_t off) { return (const char*)experts[c] + off; };
  const size_t B = L.blk0 + (size_t)l * L.blkstride;
  auto S_of = [&](int g, int c) { return gr[g].Rg * (c + 1) * p.CS; };
  auto Sr_of = [&](int c) { return (c + 1) * p.CS; };
  int rc;
  auto wargs = [&](int N, int K, int ks) {
    WArgs a = {};
    a.nex = nex; a.N = N; a.K = K; a.ks = ks; a.pair = ng > 1;
    return a;
  };
  // QKV: q, k, v = fp16(LN_self(x) W_in^T + b_in)
  {
    WArgs a = wargs(3 * d, d, 1);
    for (int g = 0; g < ng; ++g)
      for (int c = 0; c < nch; ++c) {
        WEx& x = a.ex[g * nch + c];
        x.w = (const h16x8*)PTR(c, B + L.qkv); x.a = gr[g].w.abuf[c]; x.lda = d;
        x.bias = (const h16*)PTR(c, B + L.qkv_b); x.out = gr[g].w.qkv[c]; x.S = S_of(g, c);
      }
    if ((rc = launch_wide<E_BIAS16>(a, sh.wv_qkv, st))) return rc;
  }
  // causal self attention of every (request, head), into the LN rows' buffer (free until the residual)
  {
    SelfArgs sa = {};
    sa.nex = nex; sa.H = p.H; sa.d = d; sa.hd = p.hd;
    for (int g = 0; g < ng; ++g) {
      sa.R = std::max(sa.R, gr[g].Rg);
      for (int c = 0; c < nch; ++c) {
        const int e = g * nch + c;
        sa.qkv[e] = gr[g].w.qkv[c]; sa.out[e] = gr[g].w.abuf[c]; sa.S[e] = S_of(g, c); sa.Sr[e] = Sr_of(c);
      }
    }
    if ((rc = launch_self_attn(sa, st))) return rc;
  }
  // O: out_proj, split-K partials
  {
    WArgs a = wargs(d, d, sh.ks_wo);
    for (int g = 0; g < ng; ++g)
      for (int c = 0; c < nch; ++c) {
        WEx& x = a.ex[g * nch + c];
        x.w = (const h16x8*)PTR(c, B + L.o); x.a = gr[g].w.abuf[c]; x.lda = d; x.out = gr[g].w.P[c];
        x.S = S_of(g, c);
      }
    if ((rc = launch_wide<E_PART>(a, sh.wv_split, st))) return rc;
  }
  ResArgs r = {};
  r.nex = nex; r.d = d; r.mode = p.res_mode;
  for (int g = 0; g < ng; ++g)
    for (int c = 0; c < nch; ++c) {
      const int e = g * nch + c;
      r.x[e] = gr[g].w.x[c]; r.P[e] = gr[g].w.P[c]; r.a[e] = gr[g].w.abuf[c]; r.rows[e] = S_of(g, c);
    }
  auto res_params = [&](size_t bias_off, size_t g_off, size_t b_off) {
    for (int g = 0; g < ng; ++g)
      for (int c = 0; c < nch; ++c) {
        const int e = g * nch + c;
        r.bias[e] = (const h16*)PTR(c, bias_off);
        r.g[e] = (const h16*)PTR(c, g_off); r.b[e] = (const h16*)PTR(c, b_off);
      }
  };
  // residual + LN_cross (as the folded cross attention's operand image, or plain rows)
  r.ks = sh.ks_wo;
  res_params(B + L.o_b, B + L.xn_w, B + L.xn_b);
  r.pack = p.fold;
  if ((rc = launch_res(r, st))) return rc;
  r.pack = 0;
  if (!p.fold) {
    // unfolded: q = fp16(LN_cross(x) Wq^T + bq) into the q|k|v buffer (free after the self
    // attention), attention per (request, head) over its context K/V into the LN rows' buffer,
    // out-projection split-K
    WArgs a = wargs(d, d, 1);
    for (int g = 0; g < ng; ++g)
      for (int c = 0; c < nch; ++c) {
        WEx& x = a.ex[g * nch + c];
        x.w = (const h16x8*)PTR(c, B + L.qc); x.a = gr[g].w.abuf[c]; x.lda = d;
        x.bias = (const h16*)PTR(c, B + L.qc_b); x.out = gr[g].w.qkv[c]; x.S = S_of(g, c);
      }
    if ((rc = launch_wide<E_BIAS16>(a, sh.wv_qc, st))) return rc;
    CrossArgs ca = {};
    ca.nex = nex; ca.H = p.H; ca.d = d; ca.hd = p.hd; ca.C = p.C;
    for (int g = 0; g < ng; ++g) {
      ca.R = std::max(ca.R, gr[g].Rg);
      const int Cg = gr[g].Rg * p.C;
      for (int c = 0; c < nch; ++c) {
        const int e = g * nch + c;
        ca.q[e] = gr[g].w.qkv[c]; ca.kv[e] = gr[g].w.kvc[c] + (size_t)l * 2 * Cg * d; ca.out[e] = gr[g].w.abuf[c];
        ca.S[e] = S_of(g, c); ca.Sr[e] = Sr_of(c); ca.Ct[e] = Cg;
      }
    }
    if ((rc = launch_cross_attn(ca, st))) return rc;
    WArgs o = wargs(d, d, sh.ks_oc);
    for (int g = 0; g < ng; ++g)
      for (int c = 0; c < nch; ++c) {
        WEx& x = o.ex[g * nch + c];
        x.w = (const h16x8*)PTR(c, B + L.oc); x.a = gr[g].w.abuf[c]; x.lda = d; x.out = gr[g].w.P[c];
        x.S = S_of(g, c);
      }
    if ((rc = launch_wide<E_PART>(o, sh.wv_split, st))) return rc;
  } else {
    // folded cross attention, two requests a subgroup
    XattArgs x = {};
    x.nex = nex; x.d = d; x.H = p.H; x.Cq = p.C; x.nb = p.xnb; x.scale = 1.0f / sqrtf((float)p.hd);
    x.Csg = 2 * p.C;
    for (int g = 0; g < ng; ++g) {
      const int Cg = gr[g].Rg * p.C;
      const size_t per_l = (size_t)p.H * Cg * d;
      x.C = std::max(x.C, Cg);
      x.nsg = std::max(x.nsg, (gr[g].Rg + 1) / 2);
      for (int c = 0; c < nch; ++c) {
        const int e = g * nch + c;
        const WS& w = gr[g].w;
        x.xn[e] = w.abuf[c]; x.A[e] = w.fa[c] + (size_t)l * per_l; x.Bf[e] = w.fb[c] + (size_t)l * per_l;
        x.sb[e] = w.fsb[c] + (size_t)l * p.H * Cg;
        x.out[e] = w.P[c]; x.S[e] = S_of(g, c); x.Sr[e] = Sr_of(c); x.Ssg[e] = 2 * Sr_of(c); x.Ce[e] = Cg;
      }
    }
    if ((rc = launch_xattn(x, st))) return rc;
  }
  // residual + LN_ffn (one partial per head, or the out-projection's k-splits)
  r.ks = p.fold ? p.H : sh.ks_oc;
  res_params(B + L.oc_b, B + L.fn_w, B + L.fn_b);
  if ((rc = launch_res(r, st))) return rc;
  // W1: g = fp16(gelu(LN_ffn(x) W1^T + b1))
  {
    WArgs a = wargs(fd, d, 1);
    a.gelu_r16 = p.res_mode == RES_ADD16;
    for (int g = 0; g < ng; ++g)
      for (int c = 0; c < nch; ++c) {
        WEx& x = a.ex[g * nch + c];
        x.w = (const h16x8*)PTR(c, B + L.w1); x.a = gr[g].w.abuf[c]; x.lda = d;
        x.bias = (const h16*)PTR(c, B + L.w1_b); x.out = gr[g].w.g[c]; x.S = S_of(g, c);
      }
    if ((rc = launch_wide<E_GELU16>(a, sh.wv_w1, st))) return rc;
  }
  // W2: split-K partials
  {
    WArgs a = wargs(d, fd, sh.ks_ww2);
    for (int g = 0; g < ng; ++g)
      for (int c = 0; c < nch; ++c) {
        WEx& x = a.ex[g * nch + c];
        x.w = (const h16x8*)PTR(c, B + L.w2); x.a = gr[g].w.g[c]; x.lda = fd; x.out = gr[g].w.P[c];
        x.S = S_of(g, c);
      }
    if ((rc = launch_wide<E_PART>(a, sh.wv_split, st))) return rc;
  }
  // residual + LayerNorm of the next block (out_norm after the last block)
  r.ks = sh.ks_ww2;
  if (l + 1 < NL) {
    const size_t Bn = L.blk0 + (size_t)(l + 1) * L.blkstride;
    res_params(B + L.w2_b, Bn + L.sn_w, Bn + L.sn_b);
  } else {
    res_params(B + L.w2_b, L.on_w, L.on_b);
  }
  return launch_res(r, st);
}

// Per-draft launches of `ng` wide groups: the context rows' LayerNorm of every block, the cross K/V
// of every block (context rows of every request as rows of one stream), and the folded factors.
int per_draft_wide(const Plan& p, const WideShape& sh, const cfh::ExpertLayout& L, const GroupRun* gr, int ng,
                   const void* const* experts, hipStream_t st) {
  const int d = p.d, NL = p.NL, nch = p.nch;
  auto PTR = [&](int c, size_t off) { return (const char*)experts[c] + off; };
  auto BLK = [&](int l) { return L.blk0 + (size_t)l * L.blkstride; };
  int rc;
  for (int g = 0; g < ng; ++g) {
    CtxLnArgs a = {};
    a.ctx = gr[g].ctx; a.mom = gr[g].w.ctx_mom; a.vstride = (long long)L.blkstride; a.nex = nch; a.nl = NL;
    a.Ct = gr[g].Rg * p.C; a.d = d;
    for (int c = 0; c < nch; ++c) {
      a.g0[c] = (const h16*)PTR(c, BLK(0) + L.cn_w); a.b0[c] = (const h16*)PTR(c, BLK(0) + L.cn_b);
      a.out[c] = gr[g].w.cln[c];
    }
    hipLaunchKernelGGL(k_ctx_ln, dim3(512), dim3(256), 0, st, a);
    CFH_LAUNCH_CHECK();
  }
  // cross K/V = fp16(LN_c(ctx) W_kv^T + b_kv) as [2][Cg][d] per block: per launch `per` weight sets
  // (expert, block), each once per group
  const int per = std::min(4 / ng, nch * NL);
  for (int i0 = 0; i0 < nch * NL; i0 += per) {
    WArgs a = {};
    a.N = 2 * d; a.K = d; a.ks = 1;
    const int n = std::min(per, nch * NL - i0);
    a.pair = ng > 1;
    for (int g = 0; g < ng; ++g)
      for (int i = i0; i < i0 + n; ++i) {
        const int c = i / NL, l = i - c * NL, Cg = gr[g].Rg * p.C;
        WEx& x = a.ex[a.nex++];
        x.w = (const h16x8*)PTR(c, BLK(l) + L.kv); x.a = gr[g].w.cln[c] + (size_t)l * Cg * d; x.lda = d;
        x.bias = (const h16*)PTR(c, BLK(l) + L.kv_b); x.out = gr[g].w.kvc[c] + (size_t)l * 2 * Cg * d; x.S = Cg;
        x.nsplit = d;
      }
    if ((rc = launch_wide<E_BIAS16>(a, sh.wv_kv, st))) return rc;
  }
  if (!p.fold) return CFH_OK;   // (the unfolded cross attention needs only the K/V rows)
  for (int g = 0; g < ng; ++g) {
    const int Cg = gr[g].Rg * p.C;
    XbiasArgs xb = {};
    xb.nex = nch; xb.nl = NL; xb.d = d; xb.H = p.H; xb.C = Cg;
    xb.kstride = (long long)2 * Cg * d; xb.bstride = (long long)L.blkstride;
    for (int c = 0; c < nch; ++c) {
      xb.K[c] = gr[g].w.kvc[c]; xb.bq[c] = (const h16*)PTR(c, BLK(0) + L.qc_b); xb.sb[c] = gr[g].w.fsb[c];
    }
    hipLaunchKernelGGL(k_xbias, dim3(nch * NL, (p.H * Cg + 63) / 64), dim3(1024), 0, st, xb);
    CFH_LAUNCH_CHECK();
  }
  // A_h = Wq_h^T K_h^T (the transposed query weight against the K rows) and B_h = Wo_h V_h, split-K
  // by head: the partial of k-split h, rounded to fp16, is head h's factor
  for (int l = 0; l < NL; ++l)
    for (int part = 0; part < 2; ++part) {
      // both parts of every expert in one launch when they fit the launch's four entries
      const bool both = 2 * nch * ng <= 4;
      if (both && part == 1) break;
      WArgs a = {};
      a.N = d; a.K = d; a.ks = p.H; a.pair = ng > 1;
      for (int g = 0; g < ng; ++g)
        for (int q = 0; q < 2; ++q) {
          if (!both && q != part) continue;
          const int Cg = gr[g].Rg * p.C;
          const size_t per_l = (size_t)p.H * Cg * d;
          for (int c = 0; c < nch; ++c) {
            WEx& x = a.ex[a.nex++];
            const h16* kv = gr[g].w.kvc[c] + (size_t)l * 2 * Cg * d;
            x.w = (const h16x8*)PTR(c, BLK(l) + (q == 0 ? L.qc : L.oc));
            x.a = q == 0 ? kv : kv + (size_t)Cg * d;
            x.lda = d; x.S = Cg; x.hrows = Cg;
            x.out = (q == 0 ? gr[g].w.fa[c] : gr[g].w.fb[c]) + (size_t)l * per_l;
            x.pack = q == 0;
          }
        }
      if ((rc = launch_wide<E_PART16>(a, 4, st))) return rc;
    }
  return CFH_OK;
}

// Companion streams of a caller stream: chunk expert c > 0 runs its block passes, its OUT launch
// and its Euler update on companion c-1 (default priority) for the whole draft, forked from the
// caller's stream after the per-draft launches and joined back at the end; one expert's row
// kernels, cross attention and launch gaps then overlap another's weight streaming (its launches
// half the grid of a both-experts launch).  Each companion needs a hardware queue of its own: HIP
// maps streams onto GPU_MAX_HW_QUEUES queues (4 by default), and two streams on one queue run in
// submission order.  Created on first use per (device, caller stream), only as many as the flow's
// chunk experts need, and kept for the life of the process; events are re-recorded at every step
// (a wait takes the event's state when it is enqueued), which also holds under stream capture.
constexpr int MAX_CHUNKS = 4;      // chunk experts of a flow (cfh::flow_dims_ok)
struct Companions {
  int made;                          // companions created so far
  int overlap;                       // 1: the companions' work overlaps the caller's (checked once)
  hipStream_t s[MAX_CHUNKS - 1];
  hipEvent_t fork, join[MAX_CHUNKS - 1];
  hipEvent_t up[MAX_CHUNKS - 1];     // expert c's Euler update of its chunk done (waited by c + 1)
  hipEvent_t down[MAX_CHUNKS - 1];   // expert c + 1 has read chunk c's rows (waited by c, next step)
  hipEvent_t mark[MAX_CHUNKS - 1];   // expert c's first block reached the stagger point
};
std::mutex g_comp_mu;
std::map<std::pair<int, hipStream_t>, Companions> g_comp;

// The companion check's kernel: one wave that waits `ticks` of the constant wall clock (at most
// `cap` clock reads) and records when it started and ended.
__device__ long long g_wait_stamps[8][2];
__global__ void __launch_bounds__(64) k_wait(long long ticks, long long cap, int slot) {
  const long long t0 = wall_clock64();
  long long t = t0, n = 0;
  while (t - t0 < ticks && n < cap) {
    t = wall_clock64();
    ++n;
  }
  if (threadIdx.x == 0) {
    g_wait_stamps[slot][0] = t0;
    g_wait_stamps[slot][1] = t;
  }
}

// Whether work on the companions overlaps work on the caller's stream: HIP maps a process's
// streams onto a few hardware queues, and two streams that share one run in submission order
// (measured: the d = 5120 flow at 29.4 instead of 18.7 ms a pass, and 19.6 on one stream).  A
// 200 us wait is launched on each stream at once; their wall-clock intervals overlap by most of
// that when the streams run side by side, and not at all when one waits for the other.  The
// kernels' own clocks decide, so a stall of the host between the launches (the first launch of a
// kernel loads it) does not.
int companions_overlap(hipStream_t st, const Companions& c, int n, int* overlap) {
  int dev = 0, khz = 0;
  CFH_HIP(hipGetDevice(&dev));
  CFH_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
  *overlap = 0;
  if (khz <= 0 || n < 1 || n > 7) return CFH_OK;
  const long long ticks = (long long)khz / 5, cap = 1ll << 22;
  CFH_HIP(hipEventRecord(c.fork, st));
  for (int i = 0; i < n; ++i) CFH_HIP(hipStreamWaitEvent(c.s[i], c.fork, 0));
  hipLaunchKernelGGL(k_wait, dim3(1), dim3(64), 0, st, ticks, cap, 0);
  CFH_LAUNCH_CHECK();
  for (int i = 0; i < n; ++i) {
    hipLaunchKernelGGL(k_wait, dim3(1), dim3(64), 0, c.s[i], ticks, cap, i + 1);
    CFH_LAUNCH_CHECK();
    CFH_HIP(hipEventRecord(c.join[i], c.s[i]));
    CFH_HIP(hipStreamWaitEvent(st, c.join[i], 0));
  }
  CFH_HIP(hipStreamSynchronize(st));
  long long stamps[8][2] = {};
  CFH_HIP(hipMemcpyFromSymbol(stamps, HIP_SYMBOL(g_wait_stamps), sizeof(stamps), 0, hipMemcpyDeviceToHost));
  long long lo = stamps[0][0], hi = stamps[0][1];
  for (int i = 1; i <= n; ++i) {
    lo = std::max(lo, stamps[i][0]);
    hi = std::min(hi, stamps[i][1]);
  }
  *overlap = hi - lo > ticks / 2;
  return CFH_OK;
}

// The companions of caller stream st on the current device, at least n of them; with `create`
// false nothing is created (out->made < n then says they are not there).
int companions(hipStream_t st, int n, bool create, Companions* out) {
  int dev = 0;
  CFH_HIP(hipGetDevice(&dev));
  if (n < 0 || n > MAX_CHUNKS - 1) return CFH_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_comp_mu);
  auto it = g_comp.find({dev, st});
  if (!create) {
    *out = it == g_comp.end() ? Companions{} : it->second;
    return CFH_OK;
  }
  if (it == g_comp.end()) {
    Companions c = {};
    CFH_HIP(hipEventCreateWithFlags(&c.fork, hipEventDisableTiming));
    it = g_comp.emplace(std::make_pair(dev, st), c).first;
  }
  Companions& c = it->second;
  const int made0 = c.made;
  for (; c.made < n; ++c.made) {
    const int i = c.made;
    CFH_HIP(hipStreamCreateWithFlags(&c.s[i], hipStreamNonBlocking));
    CFH_HIP(hipEventCreateWithFlags(&c.join[i], hipEventDisableTiming));
    CFH_HIP(hipEventCreateWithFlags(&c.up[i], hipEventDisableTiming));
    CFH_HIP(hipEventCreateWithFlags(&c.down[i], hipEventDisableTiming));
    CFH_HIP(hipEventCreateWithFlags(&c.mark[i], hipEventDisableTiming));
  }
  if (c.made != made0) {   // new companions: check them all against the caller's stream
    const int rc = companions_overlap(st, c, c.made, &c.overlap);
    if (rc) return rc;
  }
  *out = c;
  return CFH_OK;
}

// Destroys the companions of caller stream st on the current device (none: nothing to do).  The
// streams are destroyed after their queued work ends (hipStreamDestroy's contract).
int release_companions(hipStream_t st) {
  int dev = 0;
  CFH_HIP(hipGetDevice(&dev));
  Companions c = {};
  {
    std::lock_guard<std::mutex> lock(g_comp_mu);
    auto it = g_comp.find({dev, st});
    if (it == g_comp.end()) return CFH_OK;
    c = it->second;
    g_comp.erase(it);
  }
  for (int i = 0; i < c.made; ++i) {
    CFH_HIP(hipStreamDestroy(c.s[i]));
    CFH_HIP(hipEventDestroy(c.join[i]));
    CFH_HIP(hipEventDestroy(c.up[i]));
    CFH_HIP(hipEventDestroy(c.down[i]));
    CFH_HIP(hipEventDestroy(c.mark[i]));
  }
  if (c.fork) CFH_HIP(hipEventDestroy(c.fork));
  return CFH_OK;
}

// The whole draft of `batch` requests on workspace ws (the plan's carve() layout): per request the
// per-draft launches, then E Euler steps of L block passes and the OUT / ROWS step.
// anchor: null, or the anchored latent drafter's anchor rows [n_chunks][batch][d] fp16 (cfh_flow_anchor).
// Bytes between the two groups' workspaces of a paired wide launch sequence.
size_t group_ws_stride(const Plan& p) { return cfh::align256(carve(p, nullptr).total); }

// Workspace of a batch: one group's, or two groups' when the wide path pairs them.
size_t flow_ws_bytes(const cfh_flow_dims* dm, int batch) {
  const Plan p = make_plan(dm, group_size(dm, batch));
  if (!p.ok) return 0;
  if (p.wide && (batch + p.R - 1) / p.R > 1 && p.ws[1].ok) return 2 * group_ws_stride(p);
  return carve(p, nullptr).total;
}

// The wide path (w0: the first group's workspace): groups of p.R requests, two at a time when the
// batch has several and the paired launch shapes fit (every launch then covers both groups' rows,
// the second group's workspace after the first's).
int integrate_wide(const Plan& p, const cfh_flow_dims* dm, const cfh::ExpertLayout& L, const void* const* experts,
                   const void* ctx, void* z_out, char* ws, const WS& w0, int batch, hipStream_t st,
                   const void* anchor) {
  const int d = p.d, CS = p.CS, E = p.E, NL = p.NL, C = p.C, KD = p.KD, nch = p.nch;
  auto PTR = [&](int c, size_t off) { return (const char*)experts[c] + off; };
  auto BLK = [&](int l) { return L.blk0 + (size_t)l * L.blkstride; };
  const int ngroups = (batch + p.R - 1) / p.R;
  const int gp = ngroups > 1 && p.ws[1].ok ? 2 : 1;
  const WS w1 = gp > 1 ? carve(p, ws + group_ws_stride(p)) : w0;
  int rc;
  // the ROWS launch of a group: z0 and the step-0 rows (s < 0), or step s's Euler update
  auto rows = [&](const GroupRun& G, int s, int ks_out) {
    RowsArgs r = {};
    r.ctx = G.ctx; r.ctx_mom = G.w.ctx_mom; r.z = G.w.z; r.z_out = (h16*)z_out + (size_t)G.g0 * KD * d;
    r.d = d; r.C = C; r.CS = CS; r.nch = nch; r.KD = KD; r.R = G.Rg; r.out_all = 1; r.only = -1;
    if (s < 0) {
      r.euler = 0; r.last = 0; r.init = dm->init_mode;
    } else {
      r.euler = 1; r.last = s + 1 == E; r.ks = ks_out; r.dt = 1.0f / (float)E;
    }
    for (int c = 0; c < nch; ++c) {
      r.x[c] = G.w.x[c]; r.pos[c] = (const h16*)PTR(c, L.pos);
      r.tau[c] = (const h16*)PTR(c, L.tau) + (s < 0 ? 0 : (size_t)(s + 1 < E ? s + 1 : s) * d);
      r.g[c] = (const h16*)PTR(c, BLK(0) + L.sn_w); r.b[c] = (const h16*)PTR(c, BLK(0) + L.sn_b);
      r.a[c] = G.w.abuf[c];
      r.anchor[c] = anchor ? (const h16*)anchor + ((size_t)c * batch + G.g0) * d : nullptr;
      if (s >= 0) { r.Pout[c] = G.w.P[c]; r.bout[c] = (const h16*)PTR(c, L.out_b); }
    }
    launch_rows(r, G.Rg * KD, st);
    CFH_LAUNCH_CHECK();
    return CFH_OK;
  };
  for (int q0 = 0; q0 < ngroups; q0 += gp) {
    GroupRun gr[2];
    const int ng = std::min(gp, ngroups - q0);
    for (int g = 0; g < ng; ++g) {
      gr[g].w = g == 0 ? w0 : w1;
      gr[g].g0 = (q0 + g) * p.R;
      gr[g].Rg = std::min(p.R, batch - gr[g].g0);
      gr[g].ctx = (const h16*)ctx + (size_t)gr[g].g0 * C * d;
    }
    const WideShape& sh = p.ws[ng - 1];
    for (int g = 0; g < ng; ++g)
      if ((rc = rows(gr[g], -1, 0))) return rc;
    if ((rc = per_draft_wide(p, sh, L, gr, ng, experts, st))) return rc;
    for (int s = 0; s < E; ++s) {
      for (int l = 0; l < NL; ++l)
        if ((rc = block_pass_wide(p, sh, L, gr, ng, experts, l, st))) return rc;
      // OUT: every row of every expert (the current chunk's rows are not contiguous)
      WArgs a = {};
      a.nex = ng * nch; a.N = d; a.K = d; a.ks = sh.ks_wout; a.pair = ng > 1;
      for (int g = 0; g < ng; ++g)
        for (int c = 0; c < nch; ++c) {
          WEx& x = a.ex[g * nch + c];
          x.w = (const h16x8*)PTR(c, L.out); x.a = gr[g].w.abuf[c]; x.lda = d; x.out = gr[g].w.P[c];
          x.S = gr[g].Rg * (c + 1) * CS;
        }
      if ((rc = launch_wide<E_PART>(a, sh.wv_split, st))) return rc;
      for (int g = 0; g < ng; ++g)
        if ((rc = rows(gr[g], s, sh.ks_wout))) return rc;
    }
  }
  return CFH_OK;
}

int integrate(const Plan& p0, const cfh_flow_dims* dm, const void* const* experts, const void* ctx, void* z_out,
              void* ws_ptr, int batch, hipStream_t st, bool may_create = true, const void* anchor = nullptr) {
  // Under stream capture every expert stays on the caller's stream: a replayed graph of the
  // two-stream form ran slower than the one-stream form (d = 5120: 21.7 against 19.6 ms a flow
  // pass; d = 4096: 15.2 against 14.8), while eager calls gain from the overlap (19.0 ms).
  Plan p = p0;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  CFH_HIP(hipStreamIsCapturing(st, &cap));
  if (cap != hipStreamCaptureStatusNone) p.conc = false;
  const cfh::ExpertLayout L = cfh::expert_layout(dm);
  const WS w = carve(p, (char*)ws_ptr);
  const int d = p.d, CS = p.CS, E = p.E, NL = p.NL, C = p.C, KD = p.KD, nch = p.nch;
  int rc = CFH_OK;
  auto PTR = [&](int c, size_t off) { return (const char*)experts[c] + off; };
  auto BLK = [&](int l) { return L.blk0 + (size_t)l * L.blkstride; };
  Companions cp = {};
  if (nch > MAX_CHUNKS) return CFH_E_UNSUPPORTED;
  if (p.conc && (rc = companions(st, nch - 1, may_create, &cp))) return rc;
  // one stream when the companions would run after the caller's work, or are not there and may not
  // be created (creating a stream allocates its hardware queue)
  if (p.conc && (cp.made < nch - 1 || !cp.overlap)) p.conc = false;

  if (p.wide) return integrate_wide(p, dm, L, experts, ctx, z_out, (char*)ws_ptr, w, batch, st, anchor);

  for (int g0 = 0; g0 < batch; g0 += p.R) {
    const int Rg = std::min(p.R, batch - g0), Cg = Rg * C;     // this group's requests, context rows
    const h16* ctx_b = (const h16*)ctx + (size_t)g0 * C * d;
    h16* zo_b = (h16*)z_out + (size_t)g0 * KD * d;

    // ---- z0 and the step-0 rows
    {
      RowsArgs r = {};
      r.ctx = ctx_b; r.ctx_mom = w.ctx_mom; r.z = w.z; r.z_out = zo_b; r.euler = 0; r.last = 0; r.d = d; r.C = C;
      r.init = dm->init_mode;
      r.only = -1;
      r.CS = CS; r.nch = nch; r.KD = KD; r.R = Rg; r.out_all = p.R > 1;
      for (int c = 0; c < nch; ++c) {
        r.x[c] = w.x[c]; r.pos[c] = (const h16*)PTR(c, L.pos); r.tau[c] = (const h16*)PTR(c, L.tau);
        r.g[c] = (const h16*)PTR(c, BLK(0) + L.sn_w); r.b[c] = (const h16*)PTR(c, BLK(0) + L.sn_b);
        r.a[c] = w.abuf[c];
        r.anchor[c] = anchor ? (const h16*)anchor + ((size_t)c * batch + g0) * d : nullptr;
      }
      launch_rows(r, Rg * KD, st);
      CFH_LAUNCH_CHECK();
    }
    // ---- cross K/V of every block (once per draft), the group's context rows together
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
        x.pout = w.Pkv + (size_t)c * NL * p.ks_kv * Cg * 2 * d;
        x.mom = w.ctx_mom;
        x.rows = Cg;
        if (p.ks_kv == 1) {   // whole-K tiles: the bias and the fp16 rows written by the GEMV itself
          x.hout = w.kvc[c];
          x.hb = (const h16*)PTR(c, BLK(0) + L.kv_b);
        }
      }
      a.kvout = 1;
      if ((rc = launch_gemv<SRC_CTX>(a, p.Ct, st))) return rc;
      if (p.ks_kv > 1) {
        ReduceArgs r = {};
        r.nex = nch; r.nl = NL; r.ks = p.ks_kv; r.rows = Cg; r.N = 2 * d; r.d = d; r.kv = 1;
        r.vstride = (long long)L.blkstride;
        for (int c = 0; c < nch; ++c) {
          r.P[c] = a.ex[c].pout;
          r.b[c] = (const h16*)PTR(c, BLK(0) + L.kv_b);
          r.out[c] = w.kvc[c];
        }
        hipLaunchKernelGGL(k_reduce, dim3(1024), dim3(256), 0, st, r);
        CFH_LAUNCH_CHECK();
      }
    }
    // ---- the folded cross attention's factors of every block: A_h = Wq_h^T K_h^T from the
    // transposed query weight against the K rows, B_h = Wo_h V_h from the out-projection against
    // the V rows, each split-K by head (the partial of head h, rounded to fp16, is the factor);
    // the rows of the group's requests side by side
    if (p.fold) {
      XbiasArgs xb = {};
      xb.nex = nch; xb.nl = NL; xb.d = d; xb.H = p.H; xb.C = Cg;
      xb.kstride = (long long)2 * Cg * d; xb.bstride = (long long)L.blkstride;
      for (int c = 0; c < nch; ++c) {
        xb.K[c] = w.kvc[c]; xb.bq[c] = (const h16*)PTR(c, BLK(0) + L.qc_b); xb.sb[c] = w.fsb[c];
      }
      if (p.fold2) {   // the masked operand rows by 64 more workgroups of the same launch
        FoldMaskArgs& fm = xb.fm;
        fm.nex = nch; fm.nl = NL; fm.C = Cg; fm.d = d; fm.hd = p.hd;
        for (int c = 0; c < nch; ++c) { fm.kv[c] = w.kvc[c]; fm.out[c] = w.fm[c]; }
        xb.mask_wgs = 64;
      }
      hipLaunchKernelGGL(k_xbias, dim3(nch * NL + xb.mask_wgs), dim3(1024), 0, st, xb);
      CFH_LAUNCH_CHECK();
      // several blocks' factors a launch (block l's entries advanced by l block strides) while the
      // launch's weights stay under FOLD_LAUNCH_BYTES: the narrow widths' per-block launches are
      // bound by their fixed cost (latent width 640: 8 launches of 5.5 us became one), the widest
      // keep one block a launch (d = 5120: 210 MB a block; merged, +15 us a draft); A and B of every
      // expert together when they fit the launch's four weight sets
      constexpr size_t FOLD_LAUNCH_BYTES = 256u << 20;
      const size_t per_l = (size_t)p.H * Cg * d;
      const size_t blk_bytes = (size_t)nch * 2 * d * d * 2;
      const int lpl = (int)std::max<size_t>(1, std::min<size_t>(NL, FOLD_LAUNCH_BYTES / blk_bytes));
      for (int l0 = 0; l0 < NL; l0 += lpl)
        for (int half = 0; half < 2; ++half) {
          if (half == 1 && 2 * nch <= 4) break;
          SArgs a = {};
          a.N = d; a.K = d; a.ks = p.ks_fold; a.wpb = p.wpb_fold; a.tpw = 1; a.d = d; a.hd = p.hd;
          a.wg_per_kc = (d / 16) / a.wpb;
          a.nl = std::min(lpl, NL - l0);
          a.lwb = (long long)L.blkstride;
          a.lab = (long long)(p.fold2 ? 2 * 2 * Cg * d : 2 * Cg * d) * 2;
          a.lob = (long long)per_l * 2;
          for (int part = 0; part < 2; ++part) {
            if (2 * nch > 4 && part != half) continue;
            for (int c = 0; c < nch; ++c) {
              SEx& x = a.ex[a.nex++];
              const h16* kv = w.kvc[c] + (size_t)l0 * 2 * Cg * d;
              x.w = (const h16x8*)PTR(c, BLK(l0) + (part == 0 ? (p.fold2 ? L.qct : L.qc) : L.oc));
              if (p.fold2) {   // 2 Cg rows a k-chunk: its first head's, then its second head's
                x.a = w.fm[c] + (size_t)(l0 * 2 + part) * 2 * Cg * d;
                x.S = 2 * Cg;
              } else {
                x.a = part == 0 ? kv : kv + (size_t)Cg * d;
                x.S = Cg;
              }
              x.hrows = Cg;         // one head's factor block per Cg rows
              x.lda = d;
              x.out = (part == 0 ? w.fa[c] : w.fb[c]) + (size_t)l0 * per_l;
              x.pack = part == 0;   // A: the cross attention's score operand image
            }
          }
          if ((rc = launch_stream<S_BUF, E_PART16>(a, p.S_fold, st))) return rc;
        }
    }
    if (p.conc) {   // companions start after the per-draft launches
      CFH_HIP(hipEventRecord(cp.fork, st));
      for (int c = 1; c < nch; ++c) CFH_HIP(hipStreamWaitEvent(cp.s[c - 1], cp.fork, 0));
    }
    auto rows_args = [&](int s, int only) {
      RowsArgs r = {};
      r.ctx = ctx_b; r.z = w.z; r.z_out = zo_b; r.euler = 1; r.last = (s + 1 == E); r.ks = p.ks_out;
      r.dt = 1.0f / (float)E; r.d = d; r.C = C; r.CS = CS; r.nch = nch; r.KD = KD; r.R = Rg; r.out_all = p.R > 1;
      r.only = only;
      for (int c = 0; c < nch; ++c) {
        r.Pout[c] = w.P[c]; r.bout[c] = (const h16*)PTR(c, L.out_b);
        r.x[c] = w.x[c]; r.pos[c] = (const h16*)PTR(c, L.pos);
        r.tau[c] = (const h16*)PTR(c, L.tau) + (size_t)(s + 1 < E ? s + 1 : s) * d;
        r.g[c] = (const h16*)PTR(c, BLK(0) + L.sn_w); r.b[c] = (const h16*)PTR(c, BLK(0) + L.sn_b);
        r.a[c] = w.abuf[c];
        r.anchor[c] = anchor ? (const h16*)anchor + ((size_t)c * batch + g0) * d : nullptr;
      }
      return r;
    };
    // OUT: out_proj on the out_norm rows of experts c0 .. c0 + nc - 1's current chunks (every row
    // when requests are packed: their current rows are not contiguous, and the weights stream once
    // either way)
    auto out_proj = [&](int c0, int nc, hipStream_t sc) {
      SArgs a = {};
      a.conc = nch / nc;
      a.nex = nc; a.N = d; a.K = d; a.ks = p.ks_out; a.wpb = p.wpb_out; a.tpw = 1; a.d = d; a.hd = p.hd;
      a.wg_per_kc = (d / 16) / (a.wpb * a.tpw);
      for (int c = c0; c < c0 + nc; ++c) {
        SEx& x = a.ex[c - c0];
        x.w = (const h16x8*)PTR(c, L.out); x.lda = d; x.out = w.P[c];
        if (p.R == 1) {
          x.a = w.abuf[c] + (size_t)c * CS * d;
          x.S = CS;
        } else {
          x.a = w.abuf[c];
          x.S = Rg * (c + 1) * CS;
        }
      }
      return launch_stream<S_BUF, E_PART>(a, p.R == 1 ? CS : p.Smax, sc);
    };
    for (int s = 0; s < E; ++s) {
      if (!p.conc) {
        for (int l = 0; l < NL; ++l)
          if ((rc = block_pass(p, L, w, experts, l, Rg, st, 0, nch))) return rc;
        if ((rc = out_proj(0, nch, st))) return rc;
        const RowsArgs r = rows_args(s, -1);
        launch_rows(r, Rg * KD, st);
        CFH_LAUNCH_CHECK();
        continue;
      }
      // Each chunk expert on its own stream through the whole draft.  Expert c's next rows read
      // the rows of chunks before c, so its Euler update waits for expert c - 1's of the same
      // step (`up`), and expert c - 1 overwrites them at the next step only after expert c has
      // read them (`down`); expert 0 never waits for a later one within a step.
      // (the launches are issued block by block across the experts, so that where the host's
      // launch rate bounds the draft every stream has work queued)
      for (int l = 0; l < NL; ++l)
        for (int c = 0; c < nch; ++c) {
          hipStream_t sc = c == 0 ? st : cp.s[c - 1];
          const bool first = s == 0 && l == 0 && STAGGER_AT > 0;
          if (first && c > 0) CFH_HIP(hipStreamWaitEvent(sc, cp.mark[c - 1], 0));
          hipEvent_t mk = first && c + 1 < nch ? cp.mark[c] : nullptr;
          if ((rc = block_pass(p, L, w, experts, l, Rg, sc, c, 1, mk))) return rc;
        }
      for (int c = 0; c < nch; ++c) {
        hipStream_t sc = c == 0 ? st : cp.s[c - 1];
        if ((rc = out_proj(c, 1, sc))) return rc;
        if (c > 0) CFH_HIP(hipStreamWaitEvent(sc, cp.up[c - 1], 0));
        if (c + 1 < nch && s > 0) CFH_HIP(hipStreamWaitEvent(sc, cp.down[c], 0));
        const RowsArgs r = rows_args(s, c);
        launch_rows(r, Rg * KD, sc);
        CFH_LAUNCH_CHECK();
        if (c + 1 < nch) CFH_HIP(hipEventRecord(cp.up[c], sc));
        if (c > 0) CFH_HIP(hipEventRecord(cp.down[c - 1], sc));
      }
    }
    if (p.conc)   // the caller's stream waits for every companion (the next group reuses the workspace)
      for (int c = 1; c < nch; ++c) {
        CFH_HIP(hipEventRecord(cp.join[c - 1], cp.s[c - 1]));
        CFH_HIP(hipStreamWaitEvent(st, cp.join[c - 1], 0));
      }
  }
  return CFH_OK;
}

// The anchored latent drafter's anchor rows (TreeVAEFlowDrafter.anchor_embed then each chunk
// expert's anchor_mlp, cf/drafters/tree_flow.py:237-241, cf/drafters/chunked_flow.py:256-262, 376):
//   t1 = fp16(W_in emb[max(token, 0)] + b_in)                       [rows][d]   (anchor_in)
//   a_c = fp16(W2_c fp16(silu(fp16(W1_c t1 + b1_c))) + b2_c)       per chunk expert c
// as split-K GEMVs over at most MAXR rows a launch and their reductions.
struct AnchorPlan {
  int ks_in, ks_d;
  size_t off_P, off_t1, off_t3, total;
};

AnchorPlan anchor_plan(int d, int hidden, int nch) {
  AnchorPlan p = {};
  p.ks_in = ksplit_for(1, d / 16, hidden, MAXR);
  p.ks_d = ksplit_for(nch, d / 16, d, MAXR);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off = cfh::align256(off + bytes);
    return o;
  };
  p.off_P = take((size_t)std::max(p.ks_in, nch * p.ks_d) * MAXR * d * 4);
  p.off_t1 = take((size_t)MAXR * d * 2);
  p.off_t3 = take((size_t)nch * MAXR * d * 2);
  p.total = off;
  return p;
}

int anchor_rows(const cfh_flow_dims* dm, int hidden, const void* const* aw, const void* embed_w, const int32_t* tokens,
                int batch, void* out, void* ws, hipStream_t st) {
  const int d = dm->d, nch = dm->draft_length / dm->chunk_size;
  const AnchorPlan ap = anchor_plan(d, hidden, nch);
  float* P = (float*)((char*)ws + ap.off_P);
  h16* t1 = (h16*)((char*)ws + ap.off_t1);
  h16* t3 = (h16*)((char*)ws + ap.off_t3);
  int rc;
  for (int r0 = 0; r0 < batch; r0 += MAXR) {
    const int m = std::min(MAXR, batch - r0);
    {   // anchor_in over the gathered embedding rows
      GemvArgs a = {};
      a.nex = 1; a.nl = 1; a.ks = ap.ks_in; a.tiles = d / 16; a.N = d; a.K = hidden;
      a.ex[0].w = (const h16x8*)aw[0]; a.ex[0].a = (const h16*)embed_w; a.ex[0].lda = hidden;
      a.ex[0].ids = tokens + r0; a.ex[0].ids_stride = 1; a.ex[0].pout = P; a.ex[0].rows = m;
      if ((rc = launch_gemv<SRC_GATHER>(a, m, st))) return rc;
      ReduceArgs r = {};
      r.nex = 1; r.nl = 1; r.ks = ap.ks_in; r.rows = m; r.N = d; r.d = d;
      r.P[0] = P; r.b[0] = (const h16*)aw[1]; r.out[0] = t1;
      hipLaunchKernelGGL(k_reduce, dim3(64), dim3(256), 0, st, r);
      CFH_LAUNCH_CHECK();
    }
    for (int layer = 0; layer < 2; ++layer) {   // anchor_mlp.0 then SiLU, anchor_mlp.2; every expert at once
      GemvArgs a = {};
      a.nex = nch; a.nl = 1; a.ks = ap.ks_d; a.tiles = d / 16; a.N = d; a.K = d;
      ReduceArgs r = {};
      r.nex = nch; r.nl = 1; r.ks = ap.ks_d; r.rows = m; r.N = d; r.d = d; r.act = layer == 0;
      for (int c = 0; c < nch; ++c) {
        GemvEx& x = a.ex[c];
        x.w = (const h16x8*)aw[2 + 4 * c + 2 * layer];
        x.a = layer == 0 ? t1 : t3 + (size_t)c * MAXR * d;
        x.lda = d; x.pout = P + (size_t)c * ap.ks_d * m * d; x.rows = m;
        r.P[c] = x.pout; r.b[c] = (const h16*)aw[3 + 4 * c + 2 * layer];
        r.out[c] = layer == 0 ? t3 + (size_t)c * MAXR * d : (h16*)out + ((size_t)c * batch + r0) * d;
      }
      if ((rc = launch_gemv<SRC_BUF>(a, m, st))) return rc;
      hipLaunchKernelGGL(k_reduce, dim3(64), dim3(256), 0, st, r);
      CFH_LAUNCH_CHECK();
    }
  }
  return CFH_OK;
}

// The no-allocation entry point's workspace: one array per device, resolved to its device address
// on the first call on each device (the array's name in host code is a host-side stand-in, never a
// device address).  Its contents persist between calls; the flow writes every workspace element
// before it reads it, so nothing needs clearing.
__device__ __align__(256) unsigned char scratch[CFH_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES];

int scratch_address(void** out) {
  int dev = 0;
  CFH_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= MAX_DEVICES) return CFH_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    CFH_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) return CFH_E_HIP;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return CFH_OK;
}

}  // namespace

namespace cfh {

int tau_ks(const cfh_flow_dims* dm) {
  return ksplit_for(dm->draft_length / dm->chunk_size, dm->d / 16, dm->d, dm->flow_steps);
}

int pack_tau(const cfh_flow_dims* dm, const ExpertLayout& L, char* base, hipStream_t st) {
  const int d = dm->d, E = dm->flow_steps, ks = tau_ks(dm);
  GemvArgs a = {};
  a.nex = 1; a.nl = 1; a.ks = ks; a.tiles = d / 16; a.N = d; a.K = d; a.E = E;
  GemvEx& x = a.ex[0];
  x.w = (const h16x8*)(base + L.tw2);
  x.g0 = (const h16*)(base + L.tw0);
  x.b0 = (const h16*)(base + L.tb0);
  x.pout = (float*)(base + L.tau_p);
  x.rows = E;
  int rc;
  if ((rc = launch_gemv<SRC_TAU>(a, E, st))) return rc;
  ReduceArgs r = {};
  r.nex = 1; r.nl = 1; r.ks = ks; r.rows = E; r.N = d; r.d = d; r.kv = 0;
  r.P[0] = x.pout;
  r.b[0] = (const h16*)(base + L.tb2);
  r.out[0] = (h16*)(base + L.tau);
  hipLaunchKernelGGL(k_reduce, dim3(256), dim3(256), 0, st, r);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

}  // namespace cfh

extern "C" {

int cfh_caps(const cfh_flow_dims* dims, int batch, int64_t* ws_bytes) {
  if (!cfh::flow_dims_ok(dims) || batch < 1) return CFH_E_UNSUPPORTED;
  if (dims->d > ROWT * ROWE || dims->draft_length > MAXR) return CFH_E_UNSUPPORTED;
  const Plan p = make_plan(dims, group_size(dims, batch));
  if (!p.ok) return CFH_E_UNSUPPORTED;
  // the workspace of every batch up to `batch`: the group sizes 1, 2 (narrow), the widest single
  // group, two of them (wide group sizes grow with the batch up to WMAXR / draft_length requests;
  // a batch of several groups runs them two at a time), and the batch itself
  size_t total = flow_ws_bytes(dims, batch);
  const int wide_max = WMAXR / dims->draft_length;
  for (int b : {1, 2, wide_max, 2 * wide_max}) {
    if (b > batch) continue;
    total = std::max(total, flow_ws_bytes(dims, b));
  }
  if (ws_bytes) *ws_bytes = (int64_t)total;
  return CFH_OK;
}

int cfh_flow_group_size(const cfh_flow_dims* dims, int batch, int* requests) {
  if (!requests) return CFH_E_INVALID;
  *requests = 0;
  if (!cfh::flow_dims_ok(dims) || batch < 1) return CFH_E_UNSUPPORTED;
  if (dims->d > ROWT * ROWE || dims->draft_length > MAXR) return CFH_E_UNSUPPORTED;
  const int R = group_size(dims, batch);
  if (!make_plan(dims, R).ok) return CFH_E_UNSUPPORTED;
  *requests = R;
  return CFH_OK;
}

int cfh_flow_plan(const cfh_flow_dims* dims, int batch, int* flags) {
  if (!flags) return CFH_E_INVALID;
  *flags = 0;
  if (!cfh::flow_dims_ok(dims) || batch < 1) return CFH_E_UNSUPPORTED;
  if (dims->d > ROWT * ROWE || dims->draft_length > MAXR) return CFH_E_UNSUPPORTED;
  const Plan p = make_plan(dims, group_size(dims, batch));
  if (!p.ok) return CFH_E_UNSUPPORTED;
  *flags = (p.fold ? CFH_PLAN_FOLD : 0) | (p.fold2 ? CFH_PLAN_FOLD2 : 0) | (p.xblk ? CFH_PLAN_XBLK : 0) |
           (p.wide ? CFH_PLAN_WIDE : 0) | (p.conc ? CFH_PLAN_CONC : 0);
  return CFH_OK;
}

int cfh_flow_integrate(const cfh_flow_dims* dm, const void* const* experts, const void* ctx, void* z_out,
                       void* ws_ptr, int batch, void* stream) {
  if (!cfh::flow_dims_ok(dm) || dm->d > ROWT * ROWE || dm->draft_length > MAXR) return CFH_E_UNSUPPORTED;
  if (!experts || !ctx || !z_out || !ws_ptr || batch < 1) return CFH_E_INVALID;
  const Plan p = make_plan(dm, group_size(dm, batch));
  if (!p.ok) return CFH_E_UNSUPPORTED;
  for (int c = 0; c < p.nch; ++c)
    if (!experts[c]) return CFH_E_INVALID;
  return integrate(p, dm, experts, ctx, z_out, ws_ptr, batch, (hipStream_t)stream);
}

int cfh_flow_integrate_anchored(const cfh_flow_dims* dm, const void* const* experts, const void* ctx,
                                const void* anchor, void* z_out, void* ws_ptr, int batch, void* stream) {
  if (!cfh::flow_dims_ok(dm) || dm->d > ROWT * ROWE || dm->draft_length > MAXR) return CFH_E_UNSUPPORTED;
  if (!experts || !ctx || !anchor || !z_out || !ws_ptr || batch < 1) return CFH_E_INVALID;
  const Plan p = make_plan(dm, group_size(dm, batch));
  if (!p.ok) return CFH_E_UNSUPPORTED;
  for (int c = 0; c < p.nch; ++c)
    if (!experts[c]) return CFH_E_INVALID;
  return integrate(p, dm, experts, ctx, z_out, ws_ptr, batch, (hipStream_t)stream, true, anchor);
}

int64_t cfh_flow_anchor_ws_bytes(const cfh_flow_dims* dm, int hidden) {
  if (!cfh::flow_dims_ok(dm) || hidden < 32 || hidden % 32) return -1;
  return (int64_t)anchor_plan(dm->d, hidden, dm->draft_length / dm->chunk_size).total;
}

int cfh_flow_anchor(const cfh_flow_dims* dm, int hidden, const void* const* aw, const void* embed_w,
                    const int32_t* tokens, int batch, void* anchor, void* ws, void* stream) {
  if (!cfh::flow_dims_ok(dm) || hidden < 32 || hidden % 32 || (dm->d / 16) % WPB) return CFH_E_UNSUPPORTED;
  if (!aw || !embed_w || !tokens || !anchor || !ws || batch < 1) return CFH_E_INVALID;
  const int nch = dm->draft_length / dm->chunk_size;
  if (nch > 4) return CFH_E_UNSUPPORTED;
  for (int i = 0; i < 2 + 4 * nch; ++i)
    if (!aw[i]) return CFH_E_INVALID;
  return anchor_rows(dm, hidden, aw, embed_w, tokens, batch, anchor, ws, (hipStream_t)stream);
}

int cfh_flow_prepare_streams(const cfh_flow_dims* dm, void* stream, int* concurrent) {
  if (concurrent) *concurrent = 0;
  if (!cfh::flow_dims_ok(dm) || dm->d > ROWT * ROWE || dm->draft_length > MAXR) return CFH_E_UNSUPPORTED;
  const Plan p = make_plan(dm, 1);
  if (!p.ok) return CFH_E_UNSUPPORTED;
  if (!p.conc) return CFH_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  CFH_HIP(hipStreamIsCapturing((hipStream_t)stream, &cap));
  if (cap != hipStreamCaptureStatusNone) return CFH_E_INVALID;   // the check synchronises the stream
  Companions cp = {};
  const int rc = companions((hipStream_t)stream, p.nch - 1, true, &cp);
  if (rc) return rc;
  if (concurrent) *concurrent = cp.made >= p.nch - 1 && cp.overlap;
  return CFH_OK;
}

int cfh_flow_query_streams(void* stream, int* companions_made, int* concurrent) {
  if (!companions_made || !concurrent) return CFH_E_INVALID;
  Companions cp = {};
  const int rc = companions((hipStream_t)stream, 0, false, &cp);
  if (rc) return rc;
  *companions_made = cp.made;
  *concurrent = cp.made > 0 && cp.overlap;
  return CFH_OK;
}

int cfh_flow_release_streams(void* stream) { return release_companions((hipStream_t)stream); }

int cfh_flow_integrate_noalloc(const cfh_flow_dims* dm, const void* const* experts, const void* ctx, void* z_out,
                               int batch, void* stream) {
  if (!cfh::flow_dims_ok(dm) || dm->d > ROWT * ROWE || dm->draft_length > MAXR) return CFH_E_UNSUPPORTED;
  if (!experts || !ctx || !z_out || batch < 1) return CFH_E_INVALID;
  // narrow groups (at most two requests a weight stream): their workspace fits the scratch array
  const Plan p = make_plan(dm, group_size(dm, batch, false));
  if (!p.ok) return CFH_E_UNSUPPORTED;
  for (int c = 0; c < p.nch; ++c)
    if (!experts[c]) return CFH_E_INVALID;
  if (carve(p, nullptr).total > (size_t)CFH_NOALLOC_SCRATCH_BYTES) return CFH_E_SCRATCH;
  void* ws = nullptr;
  int rc = scratch_address(&ws);
  if (rc) return rc;
  // companion streams only if an earlier call on this caller stream created them
  return integrate(p, dm, experts, ctx, z_out, ws, batch, (hipStream_t)stream, false);
}

}  // extern "C"
