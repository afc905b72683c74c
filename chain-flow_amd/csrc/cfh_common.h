// Shared device helpers for the chain-flow MI355X (gfx950) kernels.
//
// Conventions used by every kernel in this library:
//   * wave64; MFMA v_mfma_f32_16x16x32_{f16,bf16}.  Operand layout (checked on the device):
//       A[i][k]  : lane = i + 16*(k/8), element k%8      (i = output row / activation row)
//       B[k][n]  : lane = n + 16*(k/8), element k%8      (n = weight row / output column)
//       D[i][n]  : lane = n + 16*(i/4), accumulator i%4
//   * A linear layer W[N][K] (row-major, nn.Linear layout) is PACKED so that the B fragment of
//     (n-tile t, k-step s) is 64 lanes x 16 bytes = 1 KiB contiguous:
//         packed[(t*(K/32) + s)*64 + lane] = W[16t + lane%16][32s + 8*(lane/16) .. +7]
//     so one wave streaming one n-tile reads one contiguous run of 16*K halves.
//   * fp16 rounding (r16) is round-to-nearest-even via v_cvt_f16_f32.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 h16;
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define CFH_WAVE 64

__device__ __forceinline__ f32x4 mfma_f16(h16x8 a, h16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float r16(float x) { return (float)(h16)x; }

__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// Cross-lane steps by DPP (a VALU operand modifier, a few cycles) rather than __shfl_xor, which
// lowers to ds_bpermute through the LDS unit (~100+ cycles per step, measured to dominate the
// per-head attention staged by the flow's out-projection kernels).
//   XOR1 / XOR2   quad_perm [1,0,3,2] / [2,3,0,1]   lane ^ 1 / lane ^ 2
//   HMIRROR       row_half_mirror                   lane 7 - i within each 8 lanes
//   MIRROR        row_mirror                        lane 15 - i within each 16 lanes
// After XOR1, XOR2, HMIRROR, MIRROR with a commutative, associative combine, every lane of a
// 16-lane row holds the row's result; the four rows are then combined through readlane.
enum DppCtrl { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HMIRROR = 0x141, DPP_MIRROR = 0x140 };

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float readlane_f32(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Sum over the 16 lanes of each row, in every lane of the row.
__device__ __forceinline__ float row_sum(float v) {
  v += dpp_f32<DPP_XOR1>(v);
  v += dpp_f32<DPP_XOR2>(v);
  v += dpp_f32<DPP_HMIRROR>(v);
  v += dpp_f32<DPP_MIRROR>(v);
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {   // every lane receives the total
  v = row_sum(v);
  return (readlane_f32(v, 0) + readlane_f32(v, 16)) + (readlane_f32(v, 32) + readlane_f32(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<DPP_XOR1>(v));
  v = fmaxf(v, dpp_f32<DPP_XOR2>(v));
  v = fmaxf(v, dpp_f32<DPP_HMIRROR>(v));
  v = fmaxf(v, dpp_f32<DPP_MIRROR>(v));
  return fmaxf(fmaxf(readlane_f32(v, 0), readlane_f32(v, 16)), fmaxf(readlane_f32(v, 32), readlane_f32(v, 48)));
}

// Packed index (in h16x8 units) of the B fragment for (tile, kstep) of a layer with K inputs.
__host__ __device__ __forceinline__ size_t packed_index(int tile, int kstep, int K, int lane) {
  return ((size_t)tile * (size_t)(K / 32) + (size_t)kstep) * 64 + lane;
}

// Weight-streaming MFMA loop over one packed n-tile, split in two so that the first PF fragment
// loads can be issued before the activation chunk is staged (the weights do not depend on it):
//   TileStream<PF> ts; ts.begin(wp, nsteps);  ...stage A, __syncthreads()...;  acc = ts.run(...)
//   wp   : packed fragments of this tile at the first k-step of the chunk (lane offset added here)
//   As   : LDS rows [rows][lda] (halves); lane reads row (lane&15), k-offset 8*(lane>>4) + 32*s
//   rows : number of valid A rows (<= 16); output rows >= rows hold garbage and must not be stored
// When nsteps is a multiple of PF the loads are issued unconditionally PF steps ahead, so the
// compiler keeps PF fragment loads in flight per wave (vmcnt(PF-1) waits); other step counts
// take a plain loop.
// STRIDE = distance between consecutive k-steps of one lane, in 16-byte units (64 for the packed
// layout; 4 for a row-major [rows][K] matrix read in place).  NT = non-temporal loads (packed
// weights are read once; in-place rows use plain loads so the second half of each 128-byte line
// is served from cache).
template <int PF, int STRIDE = 64, bool NT = true>
struct TileStream {
  h16x8 buf[PF];
  const h16x8* wp;
  int nsteps;
  bool piped;

  __device__ __forceinline__ h16x8 ld(size_t s) const {
    if constexpr (NT) return __builtin_nontemporal_load(wp + s * STRIDE);
    else return wp[s * STRIDE];
  }

  // w: this lane's first fragment when STRIDE != 64; the tile base (lane offset added) when 64.
  __device__ __forceinline__ void begin(const h16x8* __restrict__ w, int n) {
    wp = (STRIDE == 64) ? w + (threadIdx.x & 63) : w;
    nsteps = n;
    piped = (n >= PF) && (n % PF == 0);
    if (piped) {
#pragma unroll
      for (int p = 0; p < PF; ++p) buf[p] = ld(p);
    }
  }

  __device__ __forceinline__ f32x4 run(const h16* As, int lda, int rows, f32x4 acc) {
    const int lane = threadIdx.x & 63;
    const int row = lane & 15;
    const int kg = lane >> 4;
    // padding-row lanes read row 0; their products only reach output rows that are never stored
    const h16* arow = As + (row < rows ? row : 0) * lda + kg * 8;
    if (piped) {
      // slot p is consumed and only then refilled PF steps ahead: the ring keeps its registers
      // across iterations (a refill issued before the multiply needs a second register, and the
      // copy back at the loop edge waits for every load in flight)
      int s0 = 0;
      for (; s0 < nsteps - PF; s0 += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
          const h16x8 a = *(const h16x8*)(arow + (s0 + p) * 32);
          acc = mfma_f16(a, buf[p], acc);
          buf[p] = ld((size_t)(s0 + PF + p));
        }
      }
#pragma unroll
      for (int p = 0; p < PF; ++p) {
        const h16x8 a = *(const h16x8*)(arow + (s0 + p) * 32);
        acc = mfma_f16(a, buf[p], acc);
      }
    } else {
      for (int s = 0; s < nsteps; ++s) {
        const h16x8 b = ld((size_t)s);
        const h16x8 a = *(const h16x8*)(arow + s * 32);
        acc = mfma_f16(a, b, acc);
      }
    }
    return acc;
  }
};

// One-call form: stream nsteps k-steps of a packed tile against LDS rows.
template <int PF>
__device__ __forceinline__ f32x4 stream_tile(const h16x8* __restrict__ wp, const h16* As, int lda,
                                             int rows, int nsteps, f32x4 acc) {
  TileStream<PF> ts;
  ts.begin(wp, nsteps);
  return ts.run(As, lda, rows, acc);
}
