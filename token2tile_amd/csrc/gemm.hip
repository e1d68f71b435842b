// Skinny GEMMs of the call: the rank-32 projection (S1), the centroid scores
// (S3) and the fp64 Gram matrices of the projection fit (S0).
//
// Both MFMA kernels compute the transposed product (output features on the
// MFMA row axis, tokens on the column axis) so that a lane owns one token and
// four consecutive output features per accumulator group.
#include "t2t_common.h"
#include <type_traits>

// work-groups of one projection launch, over all heads (32 per CU)
#define T2T_PROJ_WGS 8192

// ---------------------------------------------------------------------------
// S1: out[n, 0:32] = fp16(x[n, 0:D] @ U[0:D, 0:32]), fp32 accumulation
// ---------------------------------------------------------------------------
// Persistent: up to 8192 work-groups walk the head's 32-row blocks; U is
// staged once per work-group through LDS, and each wave keeps the next
// block's x loads in flight while it multiplies and stores the current one.
template <typename T, int D>
__global__ __launch_bounds__(256) void project_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ U,
                                                      uint16_t* __restrict__ out, int N,
                                                      long long sxh, long long sxn) {
  constexpr int KS = D / 16;
  __shared__ uint16_t sU[D * 32];
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int jl = lane & 31, hh = lane >> 5;
  const uint16_t* Uh = U + (size_t)h * D * 32;
  for (int i = threadIdx.x; i < D * 32 / 8; i += 256) ((u32x4*)sU)[i] = ((const u32x4*)Uh)[i];
  __syncthreads();
  // A operand = U^T: lane supplies U[16 s + 8 hh + t][jl]
  u32x4 ua[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int t = 0; t < 4; ++t)
      ua[s][t] = (uint32_t)sU[(16 * s + 8 * hh + 2 * t) * 32 + jl] |
                 ((uint32_t)sU[(16 * s + 8 * hh + 2 * t + 1) * 32 + jl] << 16);
  // x row n of head h at x + h sxh + n sxn (elements): [H, N, D] contiguous
  // or a strided view such as the token-major [N, H, D]
  const uint16_t* xh = x + (size_t)h * sxh;
  uint16_t* oh = out + (size_t)h * N * 32;
  const int step = gridDim.x * 4 * 32;
  auto load = [&](int r0, u32x4 (&b)[KS]) {
    const int row = r0 + jl;
#pragma unroll
    for (int s = 0; s < KS; ++s) b[s] = u32x4{0u, 0u, 0u, 0u};
    if (row < N)
#pragma unroll
      for (int s = 0; s < KS; ++s) b[s] = *(const u32x4*)(xh + (size_t)row * sxn + 16 * s + 8 * hh);
  };
  int r0 = (blockIdx.x * 4 + wave) * 32;
  u32x4 bn[KS];
  if (r0 < N) load(r0, bn);
  for (; r0 < N; r0 += step) {
    u32x4 b[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) b[s] = bn[s];
    if (r0 + step < N) load(r0 + step, bn);
    const int row = r0 + jl;
    f32x16 acc = zero16();
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if constexpr (T::code == T2T_BF16) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t w = b[s][t];
          b[s][t] = (uint32_t)bf2h((uint16_t)(w & 0xffff)) | ((uint32_t)bf2h((uint16_t)(w >> 16)) << 16);
        }
      }
      acc = Mfma<F16T>::run(ua[s], b[s], acc);
    }
    if (row < N) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 o;
        o[0] = (uint32_t)f2h(acc[4 * g + 0]) | ((uint32_t)f2h(acc[4 * g + 1]) << 16);
        o[1] = (uint32_t)f2h(acc[4 * g + 2]) | ((uint32_t)f2h(acc[4 * g + 3]) << 16);
        *(u32x2*)(oh + (size_t)row * 32 + 8 * g + 4 * hh) = o;
      }
    }
  }
}

// D = 128: rows come by LDS DMA, 16 bytes per lane, four whole rows per
// instruction, into a per-wave double buffer; 16-byte chunk c of row r sits at
// chunk c ^ (r & 15), so the B-fragment reads (32 rows, one chunk each) are
// conflict free.  The fp16 outputs of a block are staged in LDS and stored as
// 1 KB contiguous runs.  Waves work alone (no work-group barrier in the loop).
// s_waitcnt immediate (gfx9) that waits for vmcnt <= n only
#define PJ_VMCNT(n) (((n) & 0xf) | (0x7 << 4) | (0xf << 8) | ((((n) >> 4) & 0x3) << 14))
typedef __attribute__((address_space(3))) void pj_lds_t;
typedef __attribute__((address_space(1))) void pj_glb_t;
template <typename T>
__global__ __launch_bounds__(256, 2) void project_lds_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ U,
                                                             uint16_t* __restrict__ out, int N,
                                                             long long sxh, long long sxn) {
  constexpr int D = 128, KS = D / 16;
  __shared__ __attribute__((aligned(1024))) uint16_t sX0[4][32 * D];
  __shared__ __attribute__((aligned(1024))) uint16_t sX1[4][32 * D];
  __shared__ __attribute__((aligned(16))) uint16_t sO[4][32 * 32];
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int jl = lane & 31, hh = lane >> 5;
  const uint16_t* Uh = U + (size_t)h * D * 32;
  // U (8 KB) staged through the first buffers, then held as fragments
  {
    uint16_t* sU = &sX0[0][0];
    for (int i = threadIdx.x; i < D * 32 / 8; i += 256) ((u32x4*)sU)[i] = ((const u32x4*)Uh)[i];
  }
  __syncthreads();
  u32x4 ua[KS];
  {
    const uint16_t* sU = &sX0[0][0];
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        ua[s][t] = (uint32_t)sU[(16 * s + 8 * hh + 2 * t) * 32 + jl] |
                   ((uint32_t)sU[(16 * s + 8 * hh + 2 * t + 1) * 32 + jl] << 16);
  }
  __syncthreads();
  const char* xh = (const char*)(x + (size_t)h * sxh);
  const size_t rowb = (size_t)sxn * 2;
  uint16_t* oh = out + (size_t)h * N * 32;
  const int step = gridDim.x * 4 * 32;
  // DMA of block r0 into buffer B: instruction i fills rows 4 i .. 4 i + 3
  auto issue = [&](int r0, auto BUF) {
    uint16_t* sb = decltype(BUF)::value ? sX1[wave] : sX0[wave];
    const int rr = lane >> 4, p = lane & 15;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 4 * i + rr;
      int row = r0 + r;
      row = row < N ? row : N - 1;
      const char* src = xh + (size_t)row * rowb + 16 * (p ^ (r & 15));
      __builtin_amdgcn_global_load_lds((const pj_glb_t*)src, (pj_lds_t*)(sb + i * 512), 16, 0, 0);
    }
  };
  auto body = [&](int r0, auto BUF) {
    const uint16_t* sb = decltype(BUF)::value ? sX1[wave] : sX0[wave];
    // the fragment reads in inline assembly: the compiler cannot tell that
    // the DMA in flight writes the other buffer and would wait for it here
    // (the explicit vmcnt waits order these reads after their own block's DMA)
    const uint32_t sbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)sb;
    u32x4 b[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s)
      asm volatile("ds_read_b128 %0, %1"
                   : "=v"(b[s])
                   : "v"(sbase + 2u * (uint32_t)(jl * D + 8 * ((2 * s + hh) ^ (jl & 15)))));
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]), "+v"(b[4]), "+v"(b[5]), "+v"(b[6]),
                   "+v"(b[7]));
    f32x16 acc = zero16();
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if constexpr (T::code == T2T_BF16) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t w = b[s][t];
          b[s][t] = (uint32_t)bf2h((uint16_t)(w & 0xffff)) | ((uint32_t)bf2h((uint16_t)(w >> 16)) << 16);
        }
      }
      acc = Mfma<F16T>::run(ua[s], b[s], acc);
    }
    // outputs through the wave's staging rows (inline assembly for the same
    // reason; one wave's LDS accesses complete in issue order)
    const uint32_t obase = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t*)sO[wave];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 o;
      o[0] = (uint32_t)f2h(acc[4 * g + 0]) | ((uint32_t)f2h(acc[4 * g + 1]) << 16);
      o[1] = (uint32_t)f2h(acc[4 * g + 2]) | ((uint32_t)f2h(acc[4 * g + 3]) << 16);
      asm volatile("ds_write_b64 %0, %1" ::"v"(obase + 2u * (uint32_t)(jl * 32 + 8 * g + 4 * hh)), "v"(o)
                   : "memory");
    }
    u32x4 ov[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      asm volatile("ds_read_b128 %0, %1"
                   : "=v"(ov[i])
                   : "v"(obase + 2u * (uint32_t)((16 * i + (lane >> 2)) * 32 + 8 * (lane & 3)))
                   : "memory");
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(ov[0]), "+v"(ov[1]));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = 16 * i + (lane >> 2);
      if (r0 + r < N) *(u32x4*)(oh + (size_t)(r0 + r) * 32 + 8 * (lane & 3)) = ov[i];
    }
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  int r0 = (blockIdx.x * 4 + wave) * 32;
  if (r0 >= N) return;
  // After the next block's 8 DMA loads are issued, "at most 8 outstanding"
  // means every older vector-memory operation of the wave has completed: the
  // current block's loads and the previous block's output stores (waiting for
  // those stores as well costs nothing measurable, and needs no assumption on
  // how loads and stores are ordered)
  issue(r0, B0{});
  for (;;) {
    // buffer 0 holds r0 (in flight); start r0 + step into buffer 1
    const bool more = r0 + step < N;
    if (more) issue(r0 + step, B1{});
    if (more) __builtin_amdgcn_s_waitcnt(PJ_VMCNT(8)); else __builtin_amdgcn_s_waitcnt(PJ_VMCNT(0));
    body(r0, B0{});
    r0 += step;
    if (!more) break;
    const bool more2 = r0 + step < N;
    if (more2) issue(r0 + step, B0{});
    if (more2) __builtin_amdgcn_s_waitcnt(PJ_VMCNT(8)); else __builtin_amdgcn_s_waitcnt(PJ_VMCNT(0));
    body(r0, B1{});
    r0 += step;
    if (!more2) break;
  }
}

template <typename T>
static int launch_project(const void* x, const void* U, void* out, int H, int N, int D,
                          long long sxh, long long sxn, hipStream_t st) {
  int gx = cdiv(N, 128);
  const int cap = (T2T_PROJ_WGS + H - 1) / H;
  if (gx > cap) gx = cap;
  dim3 grid(gx, H);
  switch (D) {
    case 128:
      hipLaunchKernelGGL((project_lds_kernel<T>), grid, dim3(256), 0, st, (const uint16_t*)x,
                         (const uint16_t*)U, (uint16_t*)out, N, sxh, sxn);
      break;
    case 64:
      hipLaunchKernelGGL((project_kernel<T, 64>), grid, dim3(256), 0, st, (const uint16_t*)x,
                         (const uint16_t*)U, (uint16_t*)out, N, sxh, sxn);
      break;
    case 32:
      hipLaunchKernelGGL((project_kernel<T, 32>), grid, dim3(256), 0, st, (const uint16_t*)x,
                         (const uint16_t*)U, (uint16_t*)out, N, sxh, sxn);
      break;
    default:
      t2t_set_error("project: D=%d not in {32, 64, 128}", D);
      return T2T_ERR_UNSUPPORTED;
  }
  T2T_LAUNCH_CHECK("project");
  return T2T_OK;
}

static int project_impl(const void* x, int x_dtype, const void* U, void* out, int H, int N, int D,
                        int r, long long sxh, long long sxn, void* stream) {
  T2T_REQUIRE(x && U && out, "project: null pointer");
  T2T_REQUIRE(H > 0 && N > 0, "project: H=%d N=%d", H, N);
  T2T_REQUIRE(r == 32, "project: rank r=%d (kernels are built for r=32)", r);
  T2T_REQUIRE(sxn >= D && sxn % 8 == 0 && sxh % 8 == 0 && sxh >= 0,
              "project: strides (%lld, %lld) must be multiples of 8 with row stride >= D", sxh, sxn);
  if (x_dtype == T2T_F16)
    return launch_project<F16T>(x, U, out, H, N, D, sxh, sxn, (hipStream_t)stream);
  if (x_dtype == T2T_BF16)
    return launch_project<BF16T>(x, U, out, H, N, D, sxh, sxn, (hipStream_t)stream);
  t2t_set_error("project: dtype %d", x_dtype);
  return T2T_ERR_ARG;
}

extern "C" int t2t_project(const void* x, int x_dtype, const void* U, void* out, int H, int N,
                           int D, int r, void* stream) {
  return project_impl(x, x_dtype, U, out, H, N, D, r, (long long)N * D, D, stream);
}

extern "C" int t2t_project_strided(const void* x, int x_dtype, const void* U, void* out, int H,
                                   int N, int D, int r, long long x_head_stride,
                                   long long x_row_stride, void* stream) {
  return project_impl(x, x_dtype, U, out, H, N, D, r, x_head_stride, x_row_stride, stream);
}

// ---------------------------------------------------------------------------
// S3: gl[n, c] = fp16(QU[n, :] . cks[c, :]), r = 32, 128-row x 128-centroid
// tiles staged through LDS so every row segment is stored as 256 B.
// The MFMA operand order here (centroids on the A side, two k-steps of 16)
// is the single definition of the fp16 score; the fused selection kernel
// uses score_block() below so its scores are bitwise the same.
// ---------------------------------------------------------------------------
#define SC_ROWS 128
#define SC_CENT 128
#define SC_PITCH (SC_CENT + 8)

// A operand fragments of 32 centroids from an LDS tile [cent][32] (pitch 32)
__device__ inline void load_cent_frag(const uint16_t* sC, int cblk, int lane, u32x4& a0, u32x4& a1) {
  const int jl = lane & 31, hh = lane >> 5;
  const uint16_t* p = sC + (cblk * 32 + jl) * 32 + 8 * hh;
  a0 = *(const u32x4*)(p);
  a1 = *(const u32x4*)(p + 16);
}

__global__ __launch_bounds__(256) void score_kernel(const uint16_t* __restrict__ QU,
                                                    const uint16_t* __restrict__ cks,
                                                    uint16_t* __restrict__ gl, int N, int CK) {
  __shared__ __attribute__((aligned(16))) uint16_t sC[SC_CENT * 32];
  __shared__ __attribute__((aligned(16))) uint16_t sO[SC_ROWS * SC_PITCH];
  const int h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int jl = lane & 31, hh = lane >> 5;
  const int r0 = blockIdx.x * SC_ROWS;
  const int row = r0 + wave * 32 + jl;
  const bool ok = row < N;
  const uint16_t* qh = QU + (size_t)h * N * 32;
  u32x4 b0 = {0u, 0u, 0u, 0u}, b1 = {0u, 0u, 0u, 0u};
  if (ok) {
    b0 = *(const u32x4*)(qh + (size_t)row * 32 + 8 * hh);
    b1 = *(const u32x4*)(qh + (size_t)row * 32 + 16 + 8 * hh);
  }
  const uint16_t* ch = cks + (size_t)h * CK * 32;
  uint16_t* gh = gl + (size_t)h * N * CK;
  for (int c0 = 0; c0 < CK; c0 += SC_CENT) {
    __syncthreads();
    // stage 128 centroids x 32 dims (8 KB): 512 vectors of 16 B
    for (int i = tid; i < SC_CENT * 4; i += 256)
      ((u32x4*)sC)[i] = ((const u32x4*)(ch + (size_t)c0 * 32))[i];
    __syncthreads();
#pragma unroll
    for (int cb = 0; cb < SC_CENT / 32; ++cb) {
      u32x4 a0, a1;
      load_cent_frag(sC, cb, lane, a0, a1);
      f32x16 acc = zero16();
      acc = Mfma<F16T>::run(a0, b0, acc);
      acc = Mfma<F16T>::run(a1, b1, acc);
      // lane holds centroids cb*32 + 8*(a/4) + 4*hh + a%4 of token wave*32 + jl
      uint16_t* orow = sO + (wave * 32 + jl) * SC_PITCH + cb * 32 + 4 * hh;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 o;
        o[0] = (uint32_t)f2h(acc[4 * g + 0]) | ((uint32_t)f2h(acc[4 * g + 1]) << 16);
        o[1] = (uint32_t)f2h(acc[4 * g + 2]) | ((uint32_t)f2h(acc[4 * g + 3]) << 16);
        *(u32x2*)(orow + 8 * g) = o;
      }
    }
    __syncthreads();
    // store 128 rows x 256 B
    for (int i = tid; i < SC_ROWS * (SC_CENT / 8); i += 256) {
      const int rr = i / (SC_CENT / 8), cc = i % (SC_CENT / 8);
      const int grow = r0 + rr;
      if (grow < N)
        __builtin_nontemporal_store(*(const u32x4*)(sO + rr * SC_PITCH + cc * 8),
                                    (u32x4*)(gh + (size_t)grow * CK + c0 + cc * 8));
    }
  }
}

extern "C" int t2t_score(const void* QU, const void* cks, void* gl, int H, int N, int CK, int r,
                         void* stream) {
  T2T_REQUIRE(QU && cks && gl, "score: null pointer");
  T2T_REQUIRE(H > 0 && N > 0, "score: H=%d N=%d", H, N);
  T2T_REQUIRE(r == 32, "score: r=%d (kernels are built for r=32)", r);
  T2T_REQUIRE(CK > 0 && CK % SC_CENT == 0, "score: CK=%d must be a multiple of %d", CK, SC_CENT);
  hipLaunchKernelGGL(score_kernel, dim3(cdiv(N, SC_ROWS), H), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)QU, (const uint16_t*)cks, (uint16_t*)gl, N, CK);
  T2T_LAUNCH_CHECK("score");
  return T2T_OK;
}

// ---------------------------------------------------------------------------
// S0: G = x^T x / N in fp64 (products of fp16 values are exact in fp64; the
// sum runs over rows in order, so the result is deterministic).
// grid (tiles, H); each work-group owns a 64 x 64 output tile.
// ---------------------------------------------------------------------------
typedef double f64x4 __attribute__((ext_vector_type(4)));
#define GR_ROWS 64      // rows staged per step
#define GR_MAXSPLIT 64  // row splits per head (partial Grams in the workspace)

// Partial Gram products on fp64 MFMA (v_mfma_f64_16x16x4_f64).  Block (s, h)
// sums rows [s R, s R + R) of head h; wave w owns the 64 x 64 quadrant
// (w / 2, w % 2) of the D x D result as 4 x 4 blocks of 16 x 16.  Rows are
// staged through LDS as fp32 (exact for fp16 values; bf16 is rounded to fp16
// first, as the reference's backend casts to fp16).  For a k-step of four
// rows, lane l holds x[n + l / 16][c + l % 16] as both the A (Xt, 16 x 4)
// and the B (X, 4 x 16) fragment of column block c, and the 16 x 16 result
// block keeps G[c_i + l / 16 + 4 r][c_j + l % 16] in register r of lane l
// (rows interleaved by four, as measured on the GPU).
// Products of fp16 values are exact in fp64, and each output sums its rows in
// a fixed order, so the result does not depend on the launch.
template <typename T>
__global__ __launch_bounds__(256) void gram_kernel(const uint16_t* __restrict__ x,
                                                   double* __restrict__ part, int N, int D, int R) {
  __shared__ float sx[GR_ROWS][128 + 4];
  const int s = blockIdx.x, h = blockIdx.y, H = gridDim.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int qi = w >> 1, qj = w & 1;
  const bool act = qi * 64 < D && qj * 64 < D;
  const int r0 = s * R;
  const int r1 = r0 + R < N ? r0 + R : N;
  f64x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f64x4{0.0, 0.0, 0.0, 0.0};
  const uint16_t* xh = x + (size_t)h * N * D;
  const int kr = lane >> 4, kc = lane & 15;
  for (int n0 = r0; n0 < r1; n0 += GR_ROWS) {
    __syncthreads();
    for (int i = tid; i < GR_ROWS * 128; i += 256) {
      const int rr = i >> 7, cc = i & 127;
      const int n = n0 + rr;
      float v = 0.f;
      if (n < r1 && cc < D) {
        const uint16_t u = xh[(size_t)n * D + cc];
        v = (T::code == T2T_BF16) ? h2f(bf2h(u)) : h2f(u);
      }
      sx[rr][cc] = v;
    }
    __syncthreads();
    if (act) {
#pragma unroll 2
      for (int k = 0; k < GR_ROWS; k += 4) {
        double a[4], b[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          a[t] = (double)sx[k + kr][64 * qi + 16 * t + kc];
          b[t] = (double)sx[k + kr][64 * qj + 16 * t + kc];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
      }
    }
  }
  if (!act) return;
  double* ph = part + ((size_t)s * H + h) * D * D;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gi = 64 * qi + 16 * i + kr + 4 * r, gj = 64 * qj + 16 * j + kc;
        if (gi < D && gj < D) ph[(size_t)gi * D + gj] = acc[i][j][r];
      }
}

// G[h] = (sum over the splits, in split order, of the partial Grams) / N
__global__ __launch_bounds__(256) void gram_reduce_kernel(const double* __restrict__ part,
                                                          double* __restrict__ G, int S, int H,
                                                          int N, int D) {
  const int h = blockIdx.y;
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= D * D) return;
  double acc = 0.0;
  for (int s = 0; s < S; ++s) acc += part[((size_t)s * H + h) * D * D + e];
  G[(size_t)h * D * D + e] = acc / (double)N;
}

static int gram_splits(int H, int N) {
  int S = (1024 + H - 1) / H;  // about 1024 work-groups
  const int maxS = (N + 4 * GR_ROWS - 1) / (4 * GR_ROWS);  // >= 4 staging steps per split
  if (S > maxS) S = maxS;
  if (S > GR_MAXSPLIT) S = GR_MAXSPLIT;
  return S < 1 ? 1 : S;
}

extern "C" size_t t2t_gram_ws_bytes(int H, int N, int D) {
  if (H <= 0 || N <= 0 || D <= 0) return 0;
  return t2t_align256((size_t)gram_splits(H, N) * H * D * D * sizeof(double));
}

extern "C" int t2t_gram(const void* x, int x_dtype, double* G, int H, int N, int D, void* ws,
                        size_t ws_bytes, void* stream) {
  T2T_REQUIRE(x && G, "gram: null pointer");
  T2T_REQUIRE(H > 0 && N > 0 && D > 0 && D <= 128, "gram: H=%d N=%d D=%d", H, N, D);
  const size_t need = t2t_gram_ws_bytes(H, N, D);
  if (!ws || ws_bytes < need) {
    t2t_set_error("gram: workspace %zu < %zu bytes", ws_bytes, need);
    return T2T_ERR_WORKSPACE;
  }
  const int S = gram_splits(H, N);
  const int R = ((N + S - 1) / S + 3) / 4 * 4;
  hipStream_t st = (hipStream_t)stream;
  double* part = (double*)ws;
  if (x_dtype == T2T_F16)
    hipLaunchKernelGGL(gram_kernel<F16T>, dim3(S, H), dim3(256), 0, st, (const uint16_t*)x, part,
                       N, D, R);
  else if (x_dtype == T2T_BF16)
    hipLaunchKernelGGL(gram_kernel<BF16T>, dim3(S, H), dim3(256), 0, st, (const uint16_t*)x, part,
                       N, D, R);
  else {
    t2t_set_error("gram: dtype %d", x_dtype);
    return T2T_ERR_ARG;
  }
  hipLaunchKernelGGL(gram_reduce_kernel, dim3((D * D + 255) / 256, H), dim3(256), 0, st, part, G,
                     S, H, N, D);
  T2T_LAUNCH_CHECK("gram");
  return T2T_OK;
}
