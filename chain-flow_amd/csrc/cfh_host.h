// Host-side helpers shared by the C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "cfhip.h"

namespace cfh {

int set_hip_error(hipError_t e);
int last_hip_error();

#define CFH_HIP(expr)                                     \
  do {                                                    \
    hipError_t _e = (expr);                               \
    if (_e != hipSuccess) return ::cfh::set_hip_error(_e); \
  } while (0)

#define CFH_LAUNCH_CHECK() CFH_HIP(hipGetLastError())

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Byte layout of one packed chunk expert (cfh_flow_pack_expert).  Vectors are fp16 copies of the
// state_dict tensors; matrices are in MFMA tile order (cfh_common.h).
struct ExpertLayout {
  size_t pos, tw0, tb0, tw2, tb2;          // position_embedding, time_mlp
  size_t blk0, blkstride;                  // block region base / stride
  // offsets inside a block region
  size_t sn_w, sn_b, qkv, qkv_b, o, o_b, xn_w, xn_b, cn_w, cn_b, qc, qc_b, kv, kv_b, oc, oc_b,
      fn_w, fn_b, w1, w1_b, w2, w2_b;
  size_t on_w, on_b, out, out_b;           // out_norm, out_proj
  size_t tau;                              // time embeddings of every Euler step, fp16 [E][d]
  size_t tau_p;                            // their split-K partials while packing, fp32 [tau_ks][E][d]
  size_t total;
  bool fold;                               // cross attention folded (xattn_fold): qc holds Wq^T
  bool fold2;                              // xattn_fold2: qct holds Wq^T beside qc
  size_t qct;                              // (fold2 only, inside a block region)
};

bool flow_dims_ok(const cfh_flow_dims* d);
// Heads per attention k-chunk: the fewest whole heads (1, 2 or 4, dividing H) whose columns make
// a multiple of 32, the MFMA k-step; 0 if none (head widths must be multiples of 8).
int heads_per_chunk(int hd, int H);
ExpertLayout expert_layout(const cfh_flow_dims* d);
// The k-chunks of the time-MLP GEMV (the split the flow plan has always used for it).
int tau_ks(const cfh_flow_dims* d);
// The time embeddings tau_s = time_mlp(s / E) of every Euler step into a packed expert image
// (fp16 [E][d] at L.tau): a function of the weights and E alone, computed once at packing instead
// of in every draft.
int pack_tau(const cfh_flow_dims* d, const ExpertLayout& L, char* base, hipStream_t st);
// Whether the flow folds the cross attention's query and output projections into per-draft
// factors of the context K/V (one head per k-chunk: head width a multiple of 32).  The packed
// layout depends on it (the query weight is stored transposed), so packing and the flow plan both
// decide by this one function of the shape.
bool xattn_fold(const cfh_flow_dims* d);
// Two heads per attention k-chunk (head widths such as 80 or 240) and 2 x ctx_rows <= 16: the flow
// folds the cross attention of single-request groups, building the factors two heads a chunk from
// operand rows masked per head; packed request groups keep the unfolded launches.  The packed
// layout then holds the query weight twice (qc as is, qct transposed).
bool xattn_fold2(const cfh_flow_dims* d);

}  // namespace cfh
