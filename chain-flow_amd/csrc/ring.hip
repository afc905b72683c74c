// The serving proposer's context ring on MI355X: FlowDrafterProposer._ring_write + _ring_gather
// (cf/vllm_plugin/flow_proposer.py:916-961).
//
// Each request slot keeps the last C target hidden states in a circular buffer ring[slot][0..C-1]
// (row C is the reference's trash row, never read here), with rpos[slot] = the next write position
// and nval[slot] = how many rows are valid (<= C).  One launch does a step for B requests, one
// workgroup per request:
//   write : rows j < Kmax of the request come from sh[start + srcoff_j] (srcoff_j = j for a chain,
//           0 then 1 + path[slot][j-1] for the accepted path of a tree), row j is kept iff
//           j < cnt && wmask, and lands at ring[slot][(rpos + j) mod C]; then
//           rpos = (rpos + add) mod C, nval = min(nval + add, C), add = wmask ? cnt : 0;
//   gather: ctx[b][j] = ring[slot][(rpos - m + t_j) mod C], t_j = min(max(j - (C - m), 0),
//           max(m - 1, 0)), m = nval: the window oldest first, front-padded by repeating the oldest
//           row (TreeFlowDrafter._context, cf/drafters/tree_flow.py:143-148).
// Every index is computed on the device from device arrays, so the step can be captured in a graph.
// Requests of one launch must use distinct slots, except rows that append nothing (cnt 0 or
// wmask 0), which only read.
#include "cfh_kernels.h"

namespace {

struct RingArgs {
  h16* ring;             // [R][C + 1][H]
  int* rpos;             // [R]
  int* nval;             // [R]
  const h16* sh;         // [T][H] hidden states of this step's sampled / verified positions
  const int* rows;       // [B] request slots
  const int* starts;     // [B] first row of each request in sh
  const int* cnt;        // [B] rows to append, or null (a gather only)
  const int* wmask;      // [B] or null (all 1): 0 = the request's ring is not written this step
  const int* path;       // [R][path_ld] or null: accepted tree path (node per depth)
  h16* ctx;              // [B][C][H] or null
  int T, C, H, Kmax, path_ld;
};

__device__ __forceinline__ void copy_row(h16* dst, const h16* src, int H) {
  for (int v = threadIdx.x; v < H / 8; v += blockDim.x) ((h16x8*)dst)[v] = ((const h16x8*)src)[v];
}

__global__ void __launch_bounds__(256) k_ring(RingArgs a) {
  const int b = blockIdx.x;
  const int slot = a.rows[b];
  const size_t rstride = (size_t)(a.C + 1) * a.H;
  h16* ring = a.ring + (size_t)slot * rstride;
  const int head = a.rpos[slot], m0 = a.nval[slot];
  const int cnt = a.cnt ? a.cnt[b] : 0, wm = a.wmask ? a.wmask[b] : 1;
  const int start = a.starts ? a.starts[b] : 0;
  for (int j = 0; j < a.Kmax; ++j) {
    if (!(wm && j < cnt)) continue;   // the reference sends these rows to the trash row
    const int off = (a.path && j > 0) ? 1 + a.path[(size_t)slot * a.path_ld + j - 1] : j;
    const int src = min(max(start + off, 0), a.T - 1);
    copy_row(ring + (size_t)((head + j) % a.C) * a.H, a.sh + (size_t)src * a.H, a.H);
  }
  __syncthreads();   // the gather below reads rows other threads of this workgroup wrote
  const int add = wm ? cnt : 0;
  const int hn = (head + add) % a.C, m = min(m0 + add, a.C);
  // a request that appends nothing leaves its slot's pointers alone: padding rows of a graph
  // bucket may point at a live slot and only read it
  if (threadIdx.x == 0 && add > 0) {
    a.rpos[slot] = hn;
    a.nval[slot] = m;
  }
  if (!a.ctx) return;
  h16* out = a.ctx + (size_t)b * a.C * a.H;
  for (int j = 0; j < a.C; ++j) {
    const int t = min(max(j - (a.C - m), 0), max(m - 1, 0));
    const int phys = ((hn - m + t) % a.C + a.C) % a.C;
    copy_row(out + (size_t)j * a.H, ring + (size_t)phys * a.H, a.H);
  }
}

}  // namespace

extern "C" int cfh_ring_step(void* ring, int32_t* rpos, int32_t* nval, int C, int H, const void* sh, int T,
                             const int32_t* rows, const int32_t* starts, const int32_t* cnt,
                             const int32_t* wmask, const int32_t* path, int path_ld, int Kmax, int B,
                             void* ctx, void* stream) {
  if (B == 0) return CFH_OK;
  if (!ring || !rpos || !nval || !rows || B < 0 || C < 1 || H <= 0 || H % 8 || Kmax < 0) return CFH_E_INVALID;
  if (cnt && Kmax > 0 && (!sh || !starts || T < 1)) return CFH_E_INVALID;
  if (path && path_ld < Kmax - 1) return CFH_E_INVALID;
  RingArgs a = {};
  a.ring = (h16*)ring; a.rpos = (int*)rpos; a.nval = (int*)nval; a.sh = (const h16*)sh; a.rows = rows;
  a.starts = starts; a.cnt = cnt; a.wmask = wmask; a.path = path; a.ctx = (h16*)ctx;
  a.T = T; a.C = C; a.H = H; a.Kmax = cnt ? Kmax : 0; a.path_ld = path_ld;
  hipLaunchKernelGGL(k_ring, dim3(B), dim3(256), 0, (hipStream_t)stream, a);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}
