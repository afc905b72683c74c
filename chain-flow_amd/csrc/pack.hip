// Weight packing (MFMA tile order) and the library's status/version entry points.
#include <stdio.h>
#include <string.h>

#include "cfh_common.h"
#include "cfh_host.h"

namespace cfh {

static thread_local int g_last_hip = 0;
int set_hip_error(hipError_t e) {
  g_last_hip = (int)e;
  return CFH_E_HIP;
}
int last_hip_error() { return g_last_hip; }

int heads_per_chunk(int hd, int H) {
  if (hd <= 0 || hd % 8 || H <= 0) return 0;
  for (int h : {1, 2, 4})
    if ((h * hd) % 32 == 0 && H % h == 0) return h;
  return 0;
}

bool flow_dims_ok(const cfh_flow_dims* d) {
  if (!d) return false;
  if (d->d <= 0 || d->d % 64 != 0 || d->d > 16384) return false;
  if (d->heads <= 0 || d->d % d->heads != 0 || !heads_per_chunk(d->d / d->heads, d->heads)) return false;
  if ((d->d / d->heads) > 1024) return false;
  if (d->ffn_mult < 1 || d->ffn_mult > 8) return false;
  if (d->layers < 1 || d->layers > 64) return false;
  if (d->ctx_rows < 2 || d->ctx_rows > 16) return false;
  if (d->chunk_size < 1 || d->draft_length < 1 || d->draft_length > 16) return false;
  if (d->draft_length % d->chunk_size != 0) return false;
  if (d->draft_length / d->chunk_size > 4) return false;
  if (d->flow_steps < 1 || d->flow_steps > 16) return false;
  if (d->numerics != CFH_FLOW_FUSED && d->numerics != CFH_FLOW_MODULES) return false;
  if (d->init_mode < CFH_INIT_DELTA || d->init_mode > CFH_INIT_GIVEN) return false;
  return true;
}

bool xattn_fold(const cfh_flow_dims* d) {
  const int hd = d->d / d->heads;
  return heads_per_chunk(hd, d->heads) == 1 && d->ctx_rows <= 16;
}

bool xattn_fold2(const cfh_flow_dims* d) {
  const int hd = d->d / d->heads;
  return heads_per_chunk(hd, d->heads) == 2 && 2 * d->ctx_rows <= 16;
}

ExpertLayout expert_layout(const cfh_flow_dims* dm) {
  const size_t d = dm->d, fd = (size_t)dm->ffn_mult * dm->d, H = 2;  // 2 bytes per element
  ExpertLayout L;
  L.fold2 = xattn_fold2(dm);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off = align256(off + bytes);
    return o;
  };
  L.pos = take(dm->draft_length * d * H);
  L.tw0 = take(d * H);
  L.tb0 = take(d * H);
  L.tb2 = take(d * H);
  L.tw2 = take(d * d * H);
  // block region
  L.blk0 = off;
  size_t b = 0;
  auto btake = [&](size_t bytes) {
    size_t o = b;
    b = align256(b + bytes);
    return o;
  };
  L.sn_w = btake(d * H);
  L.sn_b = btake(d * H);
  L.qkv_b = btake(3 * d * H);
  L.o_b = btake(d * H);
  L.xn_w = btake(d * H);
  L.xn_b = btake(d * H);
  L.cn_w = btake(d * H);
  L.cn_b = btake(d * H);
  L.qc_b = btake(d * H);
  L.kv_b = btake(2 * d * H);
  L.oc_b = btake(d * H);
  L.fn_w = btake(d * H);
  L.fn_b = btake(d * H);
  L.w1_b = btake(fd * H);
  L.w2_b = btake(d * H);
  L.qkv = btake(3 * d * d * H);
  L.o = btake(d * d * H);
  L.qc = btake(d * d * H);
  L.kv = btake(2 * d * d * H);
  L.oc = btake(d * d * H);
  L.w1 = btake(fd * d * H);
  L.w2 = btake(d * fd * H);
  L.qct = L.fold2 ? btake(d * d * H) : 0;
  L.blkstride = b;
  off = L.blk0 + b * dm->layers;
  L.on_w = take(d * H);
  L.on_b = take(d * H);
  L.out_b = take(d * H);
  L.out = take(d * d * H);
  L.tau = take((size_t)dm->flow_steps * d * H);
  L.tau_p = take((size_t)tau_ks(dm) * dm->flow_steps * d * 4);
  L.total = off;
  L.fold = xattn_fold(dm);
  return L;
}

}  // namespace cfh

// The transpose of a row-major W[k][n] in the same tile order: out holds W^T [n][k] packed, i.e.
// out[(t*(K/32)+s)*64 + lane][j] = W[32s + 8*(lane/16) + j][16t + lane%16] (K = k).  Used once per
// weight, so the strided reads do not matter.
__global__ void k_pack_linear_t(const uint16_t* __restrict__ w, int n, int k, uint4* __restrict__ out) {
  const size_t total = (size_t)n * k / 8;    // output vectors: n rows of W^T x k/8
  const int ks = k / 32;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i & 63);
    const size_t ts = i >> 6;
    const int s = (int)(ts % ks);
    const int t = (int)(ts / ks);
    const size_t col = (size_t)t * 16 + (lane & 15);          // row of W^T = column of W
    const size_t row0 = (size_t)s * 32 + 8 * (lane >> 4);     // first of 8 rows of W
    uint16_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = w[(row0 + j) * n + col];
    out[i] = make_uint4(v[0] | (unsigned)v[1] << 16, v[2] | (unsigned)v[3] << 16, v[4] | (unsigned)v[5] << 16,
                        v[6] | (unsigned)v[7] << 16);
  }
}

// out[(t*(K/32)+s)*64 + lane] = W[16t + lane%16][32s + 8*(lane/16) .. +7]
__global__ void k_pack_linear(const uint4* __restrict__ w, int n, int k, uint4* __restrict__ out) {
  const size_t total = (size_t)n * k / 8;
  const int ks = k / 32;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i & 63);
    const size_t ts = i >> 6;
    const int s = (int)(ts % ks);
    const int t = (int)(ts / ks);
    const size_t row = (size_t)t * 16 + (lane & 15);
    const size_t col = (size_t)s * 32 + 8 * (lane >> 4);
    out[i] = w[(row * k + col) / 8];
  }
}

extern "C" {

int cfh_version(void) { return 100; }

const char* cfh_error_string(int status) {
  switch (status) {
    case CFH_OK: return "ok";
    case CFH_E_INVALID: return "invalid argument";
    case CFH_E_UNSUPPORTED: return "unsupported shape";
    case CFH_E_HIP: return "HIP runtime error";
    case CFH_E_SCRATCH: return "workspace exceeds the no-allocation scratch (CFH_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown status";
  }
}

int cfh_last_hip_error(void) { return cfh::last_hip_error(); }

int cfh_pack_linear(const void* w, int n, int k, void* out, void* stream) {
  if (!w || !out || n <= 0 || k <= 0 || n % 16 || k % 32) return CFH_E_INVALID;
  const size_t total = (size_t)n * k / 8;
  int grid = (int)((total + 255) / 256);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(k_pack_linear, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const uint4*)w, n, k,
                     (uint4*)out);
  CFH_LAUNCH_CHECK();
  return CFH_OK;
}

int64_t cfh_flow_expert_bytes(const cfh_flow_dims* dims) {
  if (!cfh::flow_dims_ok(dims)) return -1;
  return (int64_t)cfh::expert_layout(dims).total;
}

int cfh_flow_pack_expert(const cfh_flow_dims* dims, const void* const* raw, int n_raw, void* packed,
                         void* stream) {
  if (!cfh::flow_dims_ok(dims)) return CFH_E_UNSUPPORTED;
  if (!raw || !packed || n_raw != 9 + 20 * dims->layers) return CFH_E_INVALID;
  for (int i = 0; i < n_raw; ++i)
    if (!raw[i]) return CFH_E_INVALID;
  const cfh::ExpertLayout L = cfh::expert_layout(dims);
  hipStream_t st = (hipStream_t)stream;
  char* base = (char*)packed;
  const size_t d = dims->d, fd = (size_t)dims->ffn_mult * dims->d;
  auto cp = [&](size_t off, const void* src, size_t elems) -> int {
    CFH_HIP(hipMemcpyAsync(base + off, src, elems * 2, hipMemcpyDeviceToDevice, st));
    return CFH_OK;
  };
  auto pk = [&](size_t off, const void* src, int n, int k) -> int {
    return cfh_pack_linear(src, n, k, base + off, stream);
  };
  int rc;
#define CFH_TRY(x) \
  if ((rc = (x)) != CFH_OK) return rc
  CFH_TRY(cp(L.pos, raw[0], dims->draft_length * d));
  CFH_TRY(cp(L.tw0, raw[1], d));
  CFH_TRY(cp(L.tb0, raw[2], d));
  CFH_TRY(pk(L.tw2, raw[3], (int)d, (int)d));
  CFH_TRY(cp(L.tb2, raw[4], d));
  for (int l = 0; l < dims->layers; ++l) {
    const void* const* r = raw + 5 + 20 * l;
    const size_t B = L.blk0 + (size_t)l * L.blkstride;
    CFH_TRY(cp(B + L.sn_w, r[0], d));
    CFH_TRY(cp(B + L.sn_b, r[1], d));
    CFH_TRY(pk(B + L.qkv, r[2], (int)(3 * d), (int)d));
    CFH_TRY(cp(B + L.qkv_b, r[3], 3 * d));
    CFH_TRY(pk(B + L.o, r[4], (int)d, (int)d));
    CFH_TRY(cp(B + L.o_b, r[5], d));
    CFH_TRY(cp(B + L.xn_w, r[6], d));
    CFH_TRY(cp(B + L.xn_b, r[7], d));
    CFH_TRY(cp(B + L.cn_w, r[8], d));
    CFH_TRY(cp(B + L.cn_b, r[9], d));
    if (L.fold) {
      // the query weight transposed: the per-draft fold computes Wq_h^T K_h^T from it
      hipLaunchKernelGGL(k_pack_linear_t, dim3(1024), dim3(256), 0, st, (const uint16_t*)r[10], (int)d, (int)d,
                         (uint4*)(base + B + L.qc));
      CFH_HIP(hipGetLastError());
    } else {
      CFH_TRY(pk(B + L.qc, r[10], (int)d, (int)d));
    }
    if (L.fold2) {
      // and transposed, for the fold of single-request groups
      hipLaunchKernelGGL(k_pack_linear_t, dim3(1024), dim3(256), 0, st, (const uint16_t*)r[10], (int)d, (int)d,
                         (uint4*)(base + B + L.qct));
      CFH_HIP(hipGetLastError());
    }
    CFH_TRY(pk(B + L.kv, (const char*)r[10] + d * d * 2, (int)(2 * d), (int)d));
    CFH_TRY(cp(B + L.qc_b, r[11], d));
    CFH_TRY(cp(B + L.kv_b, (const char*)r[11] + d * 2, 2 * d));
    CFH_TRY(pk(B + L.oc, r[12], (int)d, (int)d));
    CFH_TRY(cp(B + L.oc_b, r[13], d));
    CFH_TRY(cp(B + L.fn_w, r[14], d));
    CFH_TRY(cp(B + L.fn_b, r[15], d));
    CFH_TRY(pk(B + L.w1, r[16], (int)fd, (int)d));
    CFH_TRY(cp(B + L.w1_b, r[17], fd));
    CFH_TRY(pk(B + L.w2, r[18], (int)d, (int)fd));
    CFH_TRY(cp(B + L.w2_b, r[19], d));
  }
  const void* const* r = raw + 5 + 20 * dims->layers;
  CFH_TRY(cp(L.on_w, r[0], d));
  CFH_TRY(cp(L.on_b, r[1], d));
  CFH_TRY(pk(L.out, r[2], (int)d, (int)d));
  CFH_TRY(cp(L.out_b, r[3], d));
  CFH_TRY(cfh::pack_tau(dims, L, base, st));
#undef CFH_TRY
  return CFH_OK;
}

}  // extern "C"
