// Error plumbing, the row gather (K into key-cluster order), centroid
// finalisation and the pinned-cluster union bit.
#include "t2t_common.h"
#include <cstdarg>
#include <cstdio>

static thread_local char g_err[512] = "";

void t2t_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int t2t_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    t2t_set_error("%s: %s", what, hipGetErrorString(e));
    return T2T_ERR_LAUNCH;
  }
  return T2T_OK;
}

extern "C" const char* t2t_last_error(void) { return g_err; }
extern "C" int t2t_abi_version(void) { return 101; }

// ---------------------------------------------------------------------------
// row gather: out[h, i] = x[h, perm[h, i]]  (16-byte vectors, 16 B per lane)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gather_rows_kernel(const u32x4* __restrict__ x,
                                                          const int32_t* __restrict__ perm,
                                                          u32x4* __restrict__ out, int N,
                                                          int vec_per_row, long long total_vec) {
  const int h = blockIdx.y;
  const long long base = (long long)h * N * vec_per_row;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total_vec;
       i += (long long)gridDim.x * blockDim.x) {
    const int row = (int)(i / vec_per_row);
    const int c = (int)(i - (long long)row * vec_per_row);
    const int src = perm[(long long)h * N + row];
    out[base + i] = __builtin_nontemporal_load(&x[base + (long long)src * vec_per_row + c]);
  }
}

extern "C" int t2t_fast_gather(const void* x, int dtype, const int32_t* perm, void* out, int H,
                               int N, int D, void* stream) {
  T2T_REQUIRE(x && perm && out, "fast_gather: null pointer");
  T2T_REQUIRE(dtype == T2T_F16 || dtype == T2T_BF16, "fast_gather: dtype %d", dtype);
  T2T_REQUIRE(H > 0 && N > 0 && D > 0 && (D * 2) % 16 == 0, "fast_gather: H=%d N=%d D=%d", H,
              N, D);
  const int vpr = D * 2 / 16;
  const long long total = (long long)N * vpr;
  int gx = (int)((total + 255) / 256);
  if (gx > 4096) gx = 4096;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(gx, H), dim3(256), 0, (hipStream_t)stream,
                     (const u32x4*)x, perm, (u32x4*)out, N, vpr, total);
  T2T_LAUNCH_CHECK("fast_gather");
  return T2T_OK;
}

// ---------------------------------------------------------------------------
// ck16 = fp16(ck2); cks = fp16(fp32(ck2 * scale))
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void centroid_finalize_kernel(const float* __restrict__ ck2,
                                                                uint16_t* __restrict__ ck16,
                                                                uint16_t* __restrict__ cks,
                                                                float scale, long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x) {
    const float v = ck2[i];
    if (ck16) ck16[i] = f2h(v);
    if (cks) cks[i] = f2h(opaque(v * scale));
  }
}

extern "C" int t2t_centroid_finalize(const float* ck2, void* ck16, void* cks, float scale, int H,
                                     int CK, int r, void* stream) {
  T2T_REQUIRE(ck2, "centroid_finalize: null ck2");
  T2T_REQUIRE(H > 0 && CK > 0 && r > 0, "centroid_finalize: bad sizes");
  const long long n = (long long)H * CK * r;
  int g = (int)((n + 255) / 256);
  if (g > 2048) g = 2048;
  hipLaunchKernelGGL(centroid_finalize_kernel, dim3(g), dim3(256), 0, (hipStream_t)stream, ck2,
                     (uint16_t*)ck16, (uint16_t*)cks, scale, n);
  T2T_LAUNCH_CHECK("centroid_finalize");
  return T2T_OK;
}

// ---------------------------------------------------------------------------
// every union row gets bit CK-1 (the reserved pinned cluster)
// ---------------------------------------------------------------------------
__global__ void union_or_last_kernel(int32_t* __restrict__ unip, int rows, int words, int bit) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < rows) unip[(long long)i * words + (bit >> 5)] |= (int32_t)(1u << (bit & 31));
}

extern "C" int t2t_union_or_last(int32_t* unip, int H, int CQ, int CK, void* stream) {
  T2T_REQUIRE(unip && H > 0 && CQ > 0 && CK > 0 && CK % 32 == 0, "union_or_last: bad args");
  const int rows = H * CQ;
  hipLaunchKernelGGL(union_or_last_kernel, dim3(cdiv(rows, 256)), dim3(256), 0,
                     (hipStream_t)stream, unip, rows, CK / 32, CK - 1);
  T2T_LAUNCH_CHECK("union_or_last");
  return T2T_OK;
}
