// S2: warm-started k-means maintenance, and the init_state helpers
// (fast_assign, deterministic centroid update), for gfx950.
//
// Pipeline of one maintenance call (all deterministic):
//   prep centroids -> assign (MFMA distances + argmin) -> stable counting
//   sort of the labels (chunk histograms, column scans, ballot-ranked
//   scatter) -> per-cluster sums by one owner wave per cluster, in sorted
//   row order (exact int64 fixed point for query clusters; sequential fp32
//   for key clusters, which also writes the cluster-ordered V) -> value
//   statistics (lam, sumv).
#include "t2t_common.h"

#define KM_R 32            // rank of the projected space
#define AS_CHUNK 256       // centroids staged per LDS chunk in assign
#define SORT_CH 1024       // rows per counting-sort chunk
#define KM_MAXC 4096

static inline int pad32(int c) { return (c + 31) & ~31; }

// ---------------------------------------------------------------------------
// fast_assign (init_state).  Transposed MFMA product: centroids on the row
// axis (A), tokens on the column axis (B), so a lane owns one token and 16
// centroids per 32-centroid block, visited in ascending index order:
// d2 = |x|^2 + (cn2 - 2 x.c); key = (bits(d2) & ~m) | c, the smallest key wins.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void fast_assign_kernel(const uint16_t* __restrict__ X,
                                                          const uint16_t* __restrict__ cen,
                                                          int32_t* __restrict__ labels, int N,
                                                          int C, int ibits) {
  constexpr int KS = D / 16;
  __shared__ __attribute__((aligned(16))) uint16_t sC[AS_CHUNK * D];
  __shared__ float sN[AS_CHUNK];
  const int h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int jl = lane & 31, hh = lane >> 5;
  const int row = blockIdx.x * 128 + wave * 32 + jl;
  const bool ok = row < N;
  const uint16_t* xh = X + (size_t)h * N * D;
  u32x4 bx[KS];
  float xsq = 0.f;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    bx[s] = u32x4{0u, 0u, 0u, 0u};
    if (ok) bx[s] = *(const u32x4*)(xh + (size_t)row * D + 16 * s + 8 * hh);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float a = h2f((uint16_t)(bx[s][t] & 0xffff)), b = h2f((uint16_t)(bx[s][t] >> 16));
      xsq += a * a + b * b;
    }
  }
  xsq = half_sum(xsq);
  const uint16_t* ch = cen + (size_t)h * C * D;
  const int Cp = (C + 31) & ~31;
  int bkey = 0x7fffffff;
  const int kmask = -(1 << ibits);
  for (int c0 = 0; c0 < Cp; c0 += AS_CHUNK) {
    const int nc = (Cp - c0) < AS_CHUNK ? (Cp - c0) : AS_CHUNK;
    __syncthreads();
    // stage the chunk (padding = 0) and the squared norms in fp32, summed
    // sequentially over the dims (each square is exact)
    for (int i = tid; i < nc * D / 8; i += 256) {
      const int ci = c0 + (i * 8) / D;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (ci < C) v = ((const u32x4*)(ch + (size_t)c0 * D))[i];
      ((u32x4*)sC)[i] = v;
    }
    for (int i = tid; i < nc; i += 256) {
      const int ci = c0 + i;
      float s = 0.f;
      if (ci < C) {
        const uint16_t* cp = ch + (size_t)ci * D;
        for (int d = 0; d < D; ++d) {
          const float v = h2f(cp[d]);
          s = s + v * v;
        }
      }
      sN[i] = (ci < C) ? s : __builtin_inff();
    }
    __syncthreads();
    for (int cb = 0; cb < nc / 32; ++cb) {
      f32x16 acc = zero16();
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4 av = *(const u32x4*)(sC + (cb * 32 + jl) * D + 16 * s + 8 * hh);
        acc = Mfma<F16T>::run(av, bx[s], acc);
      }
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        const int ci = c0 + cb * 32 + 8 * (a / 4) + 4 * hh + (a % 4);
        const float cn2 = sN[cb * 32 + 8 * (a / 4) + 4 * hh + (a % 4)];
        const float d2 = xsq + (cn2 - 2.0f * acc[a]);
        int key = (__builtin_bit_cast(int, d2) & kmask) | ci;
        if (ci >= C) key = 0x7fffffff;
        bkey = key < bkey ? key : bkey;
      }
    }
  }
  const int ok2 = (int)half_partner((uint32_t)bkey);
  bkey = ok2 < bkey ? ok2 : bkey;
  if (ok && hh == 0) labels[(size_t)h * N + row] = bkey & ((1 << ibits) - 1);
}

// ---------------------------------------------------------------------------
// k-means assignment at rank 32: d = |c|^2 + x.(-2c),
// argmin, ties to the lowest index.  One 8-wave work-group per 1024 rows, four
// 32-row blocks per wave, so every centroid fragment and norm read from LDS
// feeds four MFMA chains; the centroids (-2c and |c|^2 from cen_prep_kernel)
// are staged in chunks of CMAX rows (34 KB at 512: four work-groups per CU).
// Centroid row r keeps its 16-byte chunk c at c ^ ((r >> 2) & 3), so the 32
// rows a fragment read touches fall on distinct banks.
//
// Pruning bound from a guess: the row's previous label (the label buffer's
// old contents, any value; used only when it names a centroid).  Its distance,
// summed here in fp32, plus a bound on the rounding of that sum and of the
// MFMA's own (33 terms in any order: under 2^-18 of the sum of their
// magnitudes each; 2^-16 is taken) is strictly above the MFMA distance of the
// guessed centroid, so starting the running minimum there changes no label:
// the result is still the first centroid, in visiting order, at the minimum
// MFMA distance.  A block then costs a min tree and one compare; only a block
// whose minimum improves on some lane's running minimum looks for its lowest
// index at that value.
// ---------------------------------------------------------------------------
#define AK_WAVES 8
#define AK_CHUNK 512
#define AK_RB 4
template <int CMAX>
__global__ __launch_bounds__(AK_WAVES * 64) void assign_km_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ cprep,
    const float* __restrict__ cnorm, int32_t* __restrict__ labels, int N, int C, int pin_begin,
    int pin_label, const int32_t* __restrict__ guess) {
  constexpr int D = 32;
  __shared__ __attribute__((aligned(16))) uint16_t sC[CMAX * D];
  __shared__ __attribute__((aligned(16))) float sN[CMAX];
  const int h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int jl = lane & 31, hh = lane >> 5;
  const int Cp = (C + 31) & ~31;
  const uint16_t* xh = X + (size_t)h * N * D;
  const int rbase = blockIdx.x * (AK_WAVES * 32 * AK_RB) + wave * 32 * AK_RB + jl;
  u32x4 bx[AK_RB][2];
  float best[AK_RB];
  int bidx[AK_RB];
#pragma unroll
  for (int k = 0; k < AK_RB; ++k) {
    const int row = rbase + 32 * k;
    const bool ok = row < N;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bx[k][s] = u32x4{0u, 0u, 0u, 0u};
      if (ok) bx[k][s] = *(const u32x4*)(xh + (size_t)row * D + 16 * s + 8 * hh);
    }
    // pruning bound from the row's previous label
    best[k] = __builtin_inff();
    bidx[k] = 0;
    const int g = (ok && guess) ? guess[(size_t)h * N + row] : -1;
    const bool have = g >= 0 && g < C;
    float part = 0.f, mag = 0.f;
    if (have) {
      const uint16_t* cg = cprep + ((size_t)h * C + g) * D;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4 cv = *(const u32x4*)(cg + 16 * s + 8 * hh);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float x0 = h2f((uint16_t)(bx[k][s][t] & 0xffff)), c0 = h2f((uint16_t)(cv[t] & 0xffff));
          const float x1 = h2f((uint16_t)(bx[k][s][t] >> 16)), c1 = h2f((uint16_t)(cv[t] >> 16));
          part = fmaf(x0, c0, part);
          part = fmaf(x1, c1, part);
          mag = fmaf(fabsf(x0), fabsf(c0), mag);
          mag = fmaf(fabsf(x1), fabsf(c1), mag);
        }
      }
    }
    const float opart = __builtin_bit_cast(float, half_partner(__builtin_bit_cast(uint32_t, part)));
    const float omag = __builtin_bit_cast(float, half_partner(__builtin_bit_cast(uint32_t, mag)));
    if (have) {
      const float cn = cnorm[(size_t)h * C + g];
      const float d = cn + (hh ? opart + part : part + opart);
      const float sz = fabsf(cn) + (hh ? omag + mag : mag + omag);
      best[k] = d + 0x1p-16f * sz + 0x1p-126f;
      bidx[k] = g;
    }
  }
  auto mn = [](float a, float b) { return __builtin_elementwise_minimum(a, b); };
  const u32x4* cph = (const u32x4*)(cprep + (size_t)h * C * D);
  for (int c0 = 0; c0 < Cp; c0 += CMAX) {
  const int nc = Cp - c0 < CMAX ? Cp - c0 : CMAX;
  if (c0 > 0) __syncthreads();  // every wave is done with the previous chunk
  for (int i = tid; i < nc * 4; i += AK_WAVES * 64) {
    const int r = i >> 2, c = i & 3;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (c0 + r < C) v = cph[(size_t)c0 * 4 + i];
    ((u32x4*)sC)[r * 4 + (c ^ ((r >> 2) & 3))] = v;
  }
  for (int i = tid; i < nc; i += AK_WAVES * 64)
    sN[i] = c0 + i < C ? cnorm[(size_t)h * C + c0 + i] : __builtin_inff();
  __syncthreads();
  for (int cb = 0; cb < nc / 32; ++cb) {
    const int r = cb * 32 + jl;
    const u32x4* crow = (const u32x4*)sC + r * 4;
    const u32x4 a0 = crow[(0 + hh) ^ ((r >> 2) & 3)];
    const u32x4 a1 = crow[(2 + hh) ^ ((r >> 2) & 3)];
    f32x16 init;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const float4 nv = *(const float4*)(sN + cb * 32 + 8 * gq + 4 * hh);
      init[4 * gq + 0] = nv.x;
      init[4 * gq + 1] = nv.y;
      init[4 * gq + 2] = nv.z;
      init[4 * gq + 3] = nv.w;
    }
#pragma unroll
    for (int k = 0; k < AK_RB; ++k) {
      f32x16 acc = Mfma<F16T>::run(a0, bx[k][0], init);
      acc = Mfma<F16T>::run(a1, bx[k][1], acc);
      float t8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) t8[i] = mn(acc[2 * i], acc[2 * i + 1]);
      const float bmin = mn(mn(mn(t8[0], t8[1]), mn(t8[2], t8[3])), mn(mn(t8[4], t8[5]), mn(t8[6], t8[7])));
      if (__ballot(bmin < best[k]) != 0ull) {
        if (bmin < best[k]) {
          int ia = 15;
#pragma unroll
          for (int a = 14; a >= 0; --a) ia = acc[a] == bmin ? a : ia;
          best[k] = bmin;
          bidx[k] = c0 + cb * 32 + 8 * (ia >> 2) + 4 * hh + (ia & 3);
        }
      }
    }
  }
  }
#pragma unroll
  for (int k = 0; k < AK_RB; ++k) {
    const float ob = __builtin_bit_cast(float, half_partner(__builtin_bit_cast(uint32_t, best[k])));
    const int oi = (int)half_partner((uint32_t)bidx[k]);
    int lab = bidx[k];
    if (ob < best[k] || (ob == best[k] && oi < bidx[k])) lab = oi;
    const int row = rbase + 32 * k;
    if (row < N && hh == 0) labels[(size_t)h * N + row] = row >= pin_begin ? pin_label : lab;
  }
}

// ---------------------------------------------------------------------------
// stable counting sort of labels -> counts, cbase (exclusive scan), perm
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void sort_hist_kernel(const int32_t* __restrict__ lab,
                                                        int32_t* __restrict__ chist, int N, int C,
                                                        int nChunk) {
  __shared__ int hist[KM_MAXC];
  const int h = blockIdx.y, k = blockIdx.x, tid = threadIdx.x;
  for (int i = tid; i < C; i += 256) hist[i] = 0;
  __syncthreads();
  const int r0 = k * SORT_CH;
  const int r1 = (r0 + SORT_CH) < N ? (r0 + SORT_CH) : N;
  for (int r = r0 + tid; r < r1; r += 256) atomicAdd(&hist[lab[(size_t)h * N + r]], 1);
  __syncthreads();
  int32_t* out = chist + ((size_t)h * nChunk + k) * C;
  for (int i = tid; i < C; i += 256) out[i] = hist[i];
}

// chunk-local start offsets: chist[h, k, c] <- sum of chist[h, k', c] over
// k' < k, and counts[h, c] <- the column total.  One wave per 64 clusters,
// lane = cluster; the chunks are read 16 at a time (all in flight together),
// so the latency is a few memory round trips, not one per chunk.
#define SCAN_GRP 16
__global__ __launch_bounds__(64) void sort_colscan_kernel(int32_t* __restrict__ chist,
                                                          int32_t* __restrict__ counts, int C,
                                                          int nChunk) {
  const int h = blockIdx.y, c = blockIdx.x * 64 + threadIdx.x;
  if (c >= C) return;
  int32_t* col = chist + (size_t)h * nChunk * C + c;
  int run = 0;
  for (int k0 = 0; k0 < nChunk; k0 += SCAN_GRP) {
    int v[SCAN_GRP];
#pragma unroll
    for (int i = 0; i < SCAN_GRP; ++i) v[i] = k0 + i < nChunk ? col[(size_t)(k0 + i) * C] : 0;
#pragma unroll
    for (int i = 0; i < SCAN_GRP; ++i) {
      if (k0 + i < nChunk) col[(size_t)(k0 + i) * C] = run;
      run += v[i];
    }
  }
  counts[(size_t)h * C + c] = run;
}

__device__ inline void wave_sync_km() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// One wave per chunk of SORT_CH rows; rows of equal label keep their order
// (ballot ranking).  A cluster's start in the permutation is cbase (the
// exclusive scan of the counts over clusters) plus the chunk-local offset.
// The chunk's labels are loaded up front, so the ranking loop waits on no
// global load.
#define SC_PER (SORT_CH / 64)
__global__ __launch_bounds__(64) void sort_scatter_kernel(const int32_t* __restrict__ lab,
                                                          const int32_t* __restrict__ chist,
                                                          const int32_t* __restrict__ cbase,
                                                          int32_t* __restrict__ perm, int N, int C,
                                                          int nChunk, int lbits) {
  extern __shared__ int cc[];  // C entries
  const int h = blockIdx.y, k = blockIdx.x, l = threadIdx.x;
  const int r0 = k * SORT_CH;
  const int r1 = (r0 + SORT_CH) < N ? (r0 + SORT_CH) : N;
  int labs[SC_PER];
#pragma unroll
  for (int i = 0; i < SC_PER; ++i) {
    const int row = r0 + 64 * i + l;
    labs[i] = row < r1 ? lab[(size_t)h * N + row] : 0;
  }
  const int32_t* off = chist + ((size_t)h * nChunk + k) * C;
  const int32_t* cb = cbase + (size_t)h * C;
  for (int c = l; c < C; c += 64) cc[c] = cb[c] + off[c];
  wave_sync_km();
  const unsigned long long lt = (1ull << l) - 1ull;
#pragma unroll
  for (int i = 0; i < SC_PER; ++i) {
    const int row = r0 + 64 * i + l;
    if (r0 + 64 * i >= r1) break;  // wave-uniform
    const bool valid = row < r1;
    const int c = labs[i];
    unsigned long long peers = __ballot(valid);
    for (int b = 0; b < lbits; ++b) {
      const unsigned long long bb = __ballot((c >> b) & 1);
      peers &= ((c >> b) & 1) ? bb : ~bb;
    }
    const int rank = __popcll(peers & lt);
    const int leader = (int)__ffsll((long long)peers) - 1;
    int base = 0;
    if (valid && l == leader) {
      base = cc[c];
      cc[c] = base + __popcll(peers);
    }
    base = __shfl(base, leader < 0 ? 0 : leader, 64);
    if (valid) perm[(size_t)h * N + base + rank] = row;
    wave_sync_km();
  }
}

// cbase[h, c] = exclusive scan of counts[h, :] over clusters
__global__ __launch_bounds__(1024) void cbase_kernel(const int32_t* __restrict__ counts,
                                                     int32_t* __restrict__ cbase, int C) {
  __shared__ int wsum[16];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int per = (C + 1023) / 1024;
  int loc = 0;
  for (int i = 0; i < per; ++i) {
    const int c = tid * per + i;
    if (c < C) loc += counts[(size_t)h * C + c];
  }
  const int inc = wave_incl_scan(loc);
  if (lane == 63) wsum[w] = inc;
  __syncthreads();
  int run = inc - loc;
  for (int i = 0; i < w; ++i) run += wsum[i];
  for (int i = 0; i < per; ++i) {
    const int c = tid * per + i;
    if (c < C) {
      cbase[(size_t)h * C + c] = run;
      run += counts[(size_t)h * C + c];
    }
  }
}

struct SortBufs {
  int32_t* chist;  // [H, nChunk, C]
};

static int run_sort(const int32_t* lab, int32_t* counts, int32_t* cbase, int32_t* perm,
                    int32_t* chist, int H, int N, int C, hipStream_t st) {
  const int nChunk = cdiv(N, SORT_CH);
  int lbits = 1;
  while ((1 << lbits) < C) ++lbits;
  hipLaunchKernelGGL(sort_hist_kernel, dim3(nChunk, H), dim3(256), 0, st, lab, chist, N, C, nChunk);
  hipLaunchKernelGGL(sort_colscan_kernel, dim3(cdiv(C, 64), H), dim3(64), 0, st, chist, counts, C,
                     nChunk);
  hipLaunchKernelGGL(cbase_kernel, dim3(H), dim3(1024), 0, st, counts, cbase, C);
  hipLaunchKernelGGL(sort_scatter_kernel, dim3(nChunk, H), dim3(64), (size_t)C * sizeof(int), st,
                     lab, chist, cbase, perm, N, C, nChunk, lbits);
  return t2t_check_launch("counting sort");
}

// ---------------------------------------------------------------------------
// per-cluster integer sums in sorted order -> fp16 means (one wave/cluster)
//   MODE 0: rne(x * 32768) sums, mean = fp16(f32(S) / (32768 * f32(n)))
//   MODE 1: rne(x * 2^20) sums, mean = fp16(f32(f64(S) / 2^20 / f64(n)))
// empty clusters keep `old`.
// ---------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(256) void fixed_mean_kernel(const uint16_t* __restrict__ X,
                                                         const int32_t* __restrict__ perm,
                                                         const int32_t* __restrict__ counts,
                                                         const int32_t* __restrict__ cbase,
                                                         const uint16_t* __restrict__ old,
                                                         uint16_t* __restrict__ out, int N, int C) {
  const int h = blockIdx.y;
  const int l = threadIdx.x & 63;
  const int c = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (c >= C) return;
  const int n = counts[(size_t)h * C + c];
  const int b = cbase[(size_t)h * C + c];
  // lane l sums dims 4 (l % 8) .. + 3 of rows i with i % 8 = l / 8: the
  // cluster's row indices are read 64 at a time (one coalesced load) and
  // broadcast, so eight independent row loads are in flight per lane.  The
  // sums are exact integers, so their order does not change the result.
  const int dq = l & 7, rg = l >> 3;
  const float scale = MODE == 0 ? 32768.0f : 1048576.0f;
  long long S[4] = {0, 0, 0, 0};
  const int32_t* ph = perm + (size_t)h * N + b;
  const uint16_t* xh = X + (size_t)h * N * KM_R + 4 * dq;
  for (int i0 = 0; i0 < n; i0 += 64) {
    const int myrow = i0 + l < n ? ph[i0 + l] : -1;
    u32x2 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = __shfl(myrow, 8 * j + rg, 64);
      v[j] = row >= 0 ? *(const u32x2*)(xh + (size_t)row * KM_R) : u32x2{0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t x = (uint16_t)(v[j][e >> 1] >> (16 * (e & 1)));
        S[e] += (long long)rintf(h2f(x) * scale);
      }
  }
  // sum over the eight row groups (lane bits 3..5)
#pragma unroll
  for (int m = 8; m < 64; m <<= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) S[e] += __shfl_xor(S[e], m, 64);
  if (rg == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const size_t o = ((size_t)h * C + c) * KM_R + 4 * dq + e;
      uint16_t v;
      if (n == 0) {
        v = old[o];
      } else if (MODE == 0) {
        v = f2h(opaque((float)S[e] / (32768.0f * (float)n)));
      } else {
        const double m = ((double)S[e] / 1048576.0) / (double)n;
        v = f2h(opaque((float)m));
      }
      out[o] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// key side: per cluster, sequential fp32 sums of KU (lanes 0..31, one dim
// each) and V (two dims per lane) in sorted row order; V_sorted rows; ck2.
// perm == nullptr: rows are already cluster ordered (V_sorted input).
// ---------------------------------------------------------------------------
#define KG_UNR 16
template <typename T>
__global__ __launch_bounds__(256) void key_gather_kernel(
    const uint16_t* __restrict__ KU, const uint16_t* __restrict__ V,
    const int32_t* __restrict__ perm, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ cbase, const uint16_t* __restrict__ ck0, float* __restrict__ ck2,
    uint16_t* __restrict__ V_sorted, float* __restrict__ vsum, float* __restrict__ cmax, int N,
    int C, long long svh, long long svn) {
  const int h = blockIdx.y;
  const int l = threadIdx.x & 63;
  const int c = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (c >= C) return;
  const int n = counts[(size_t)h * C + c];
  const int b = cbase[(size_t)h * C + c];
  const int32_t* ph = perm ? perm + (size_t)h * N + b : nullptr;
  const uint16_t* kh = KU ? KU + (size_t)h * N * KM_R : nullptr;
  // V row n of head h at V + h svh + n svn (elements; svn even)
  const uint32_t* vh = (const uint32_t*)(V + (size_t)h * svh);
  const size_t vrow = (size_t)(svn >> 1);
  uint32_t* vsh = V_sorted ? (uint32_t*)(V_sorted + (size_t)h * N * 128) : nullptr;
  // lanes 0..15 also sum the projected key rows, dims 2 l and 2 l + 1 (one
  // 4-byte load per row; each dim still sums its rows in order)
  float ax0 = 0.f, ax1 = 0.f, v0 = 0.f, v1 = 0.f;
  const uint32_t* kh32 = (const uint32_t*)kh;
  // The cluster's row indices are read 64 at a time (one coalesced load) and
  // taken lane by lane as wave-uniform values, so each row's loads address
  // from a scalar base.  Rows go in chunks of KG_UNR, software pipelined:
  // chunk i + 1's loads are in flight while chunk i is stored and summed.
  // Every load is unconditional (rows past the block repeat its last row and
  // are not consumed), so the memory-counter waits can count on them.
  auto run = [&](auto KS) {
    constexpr bool ks = decltype(KS)::value;
    int nxt = (l < n) ? (ph ? ph[l] : b + l) : 0;
    for (int i0 = 0; i0 < n; i0 += 64) {
      const int myrow = nxt;
      nxt = (i0 + 64 + l < n) ? (ph ? ph[i0 + 64 + l] : b + i0 + 64 + l) : 0;
      const int m = n - i0 < 64 ? n - i0 : 64;
      uint32_t va[2][KG_UNR], xa[2][KG_UNR];
      auto load = [&](int i, uint32_t (&vv)[KG_UNR], uint32_t (&xv)[KG_UNR]) {
#pragma unroll
        for (int u = 0; u < KG_UNR; ++u) {
          const int rw = __builtin_amdgcn_readlane(myrow, i + u < m ? i + u : m - 1);
          vv[u] = __builtin_nontemporal_load(&vh[(size_t)rw * vrow + l]);
          if constexpr (ks) xv[u] = kh32[(size_t)rw * (KM_R / 2) + (l & 15)];
        }
      };
      auto consume = [&](int i, const uint32_t (&vv)[KG_UNR], const uint32_t (&xv)[KG_UNR]) {
#pragma unroll
        for (int u = 0; u < KG_UNR; ++u) {
          if (i + u >= m) break;
          if (vsh) vsh[(size_t)(b + i0 + i + u) * 64 + l] = vv[u];
          v0 += T::to_f((uint16_t)(vv[u] & 0xffff));
          v1 += T::to_f((uint16_t)(vv[u] >> 16));
          if constexpr (ks) {
            ax0 += h2f((uint16_t)(xv[u] & 0xffff));
            ax1 += h2f((uint16_t)(xv[u] >> 16));
          }
        }
      };
      load(0, va[0], xa[0]);
      for (int i = 0; i < m; i += 2 * KG_UNR) {
        load(i + KG_UNR, va[1], xa[1]);
        consume(i, va[0], xa[0]);
        if (i + KG_UNR >= m) break;
        if (i + 2 * KG_UNR < m) load(i + 2 * KG_UNR, va[0], xa[0]);
        consume(i + KG_UNR, va[1], xa[1]);
      }
    }
  };
  if (kh32)
    run(std::true_type{});
  else
    run(std::false_type{});
  float* vo = vsum + ((size_t)h * C + c) * 128 + 2 * l;
  vo[0] = v0;
  vo[1] = v1;
  // the cluster's largest |value sum|, for the per-head scale lam
  const float mx = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
  if (l == 0) cmax[(size_t)h * C + c] = mx;
  if (ck2 && l < 16) {
    const size_t o = ((size_t)h * C + c) * KM_R + 2 * l;
    ck2[o] = n ? ax0 / (float)n : h2f(ck0[o]);
    ck2[o + 1] = n ? ax1 / (float)n : h2f(ck0[o + 1]);
  }
}

// lam = max(1, max|vsum| / 32768); sumv = fp16(vsum * (1 / lam)).  The grid
// spans every head's 128 C values (VS_PER per thread): each block reduces the
// head's C per-cluster maxima (cmax, written by key_gather_kernel) to lam
// itself, so the head needs no single-block pass over all of vsum.
#define VS_PER 8
__global__ __launch_bounds__(1024) void vstats_kernel(const float* __restrict__ vsum,
                                                      const float* __restrict__ cmax,
                                                      uint16_t* __restrict__ sumv,
                                                      float* __restrict__ lam, int C) {
  __shared__ float red[16];
  const int h = blockIdx.y, tid = threadIdx.x;
  const float* ch = cmax + (size_t)h * C;
  float mx = 0.f;
  for (int i = tid; i < C; i += 1024) mx = fmaxf(mx, ch[i]);
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  mx = 0.f;
  for (int i = 0; i < 16; ++i) mx = fmaxf(mx, red[i]);
  const float lm = fmaxf(1.0f, mx / 32768.0f);
  const float inv = 1.0f / lm;
  if (blockIdx.x == 0 && tid == 0) lam[h] = lm;
  const size_t CE = (size_t)C * 128;
  const size_t i0 = ((size_t)blockIdx.x * 1024 + tid) * VS_PER;
  const float* vh = vsum + (size_t)h * CE;
  uint16_t* sh = sumv + (size_t)h * CE;
  if (i0 + VS_PER <= CE) {  // CE is a multiple of 128: every group is whole
    const f32x4 a = *(const f32x4*)(vh + i0), b = *(const f32x4*)(vh + i0 + 4);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      o[e] = (uint32_t)f2h(opaque(a[2 * e] * inv)) | ((uint32_t)f2h(opaque(a[2 * e + 1] * inv)) << 16);
      o[2 + e] = (uint32_t)f2h(opaque(b[2 * e] * inv)) | ((uint32_t)f2h(opaque(b[2 * e + 1] * inv)) << 16);
    }
    *(u32x4*)(sh + i0) = o;
  }
}
static void launch_vstats(const float* vsum, const float* cmax, void* sumv, float* lam, int H,
                          int C, hipStream_t st) {
  hipLaunchKernelGGL(vstats_kernel, dim3(cdiv(C * 128, 1024 * VS_PER), H), dim3(1024), 0, st,
                     vsum, cmax, (uint16_t*)sumv, lam, C);
}

// ---------------------------------------------------------------------------
// host entry points
// ---------------------------------------------------------------------------
struct KmmWs {
  int32_t* qlab1;
  uint16_t* cq1;
  int32_t* perm1;
  int32_t* counts1;
  int32_t* cbase1;
  int32_t* cbaseq;
  int32_t* cbasek;
  int32_t* chist;
  float* vsum;
  float* cmax;
  uint16_t* cprep;  // -2c of the centroids of the assignment in flight
  float* cnorm;     // and their squared norms
  size_t total;
};

static KmmWs kmm_layout(int H, int N, int CQ, int CK, void* base) {
  WsCarver w(base);
  KmmWs k;
  const int nChunk = cdiv(N, SORT_CH);
  const int Cmax = CQ > CK ? CQ : CK;
  k.qlab1 = w.take<int32_t>((size_t)H * N);
  k.cq1 = w.take<uint16_t>((size_t)H * CQ * KM_R);
  k.perm1 = w.take<int32_t>((size_t)H * N);
  k.counts1 = w.take<int32_t>((size_t)H * CQ);
  k.cbase1 = w.take<int32_t>((size_t)H * CQ);
  k.cbaseq = w.take<int32_t>((size_t)H * CQ);
  k.cbasek = w.take<int32_t>((size_t)H * CK);
  k.chist = w.take<int32_t>((size_t)H * nChunk * Cmax);
  k.vsum = w.take<float>((size_t)H * CK * 128);
  k.cmax = w.take<float>((size_t)H * CK);
  k.cprep = w.take<uint16_t>((size_t)H * Cmax * KM_R);
  k.cnorm = w.take<float>((size_t)H * Cmax);
  k.total = w.off;
  return k;
}

extern "C" size_t t2t_kmm_ws_bytes(int H, int N, int CQ, int CK) {
  return kmm_layout(H, N, CQ, CK, nullptr).total;
}

// -2c (exact in fp16) and the fp32 squared norm of every centroid, summed
// sequentially over the dims (each square is exact): the operands of
// assign_km_kernel
__global__ __launch_bounds__(256) void cen_prep_kernel(const uint16_t* __restrict__ cen,
                                                       uint16_t* __restrict__ cprep,
                                                       float* __restrict__ cnorm, int C) {
  const int h = blockIdx.y, ci = blockIdx.x * 256 + threadIdx.x;
  if (ci >= C) return;
  const uint16_t* cp = cen + ((size_t)h * C + ci) * KM_R;
  uint16_t* op = cprep + ((size_t)h * C + ci) * KM_R;
  float s = 0.f;
  for (int d = 0; d < KM_R; ++d) {
    const float v = h2f(cp[d]);
    s = s + v * v;
    op[d] = f2h(-2.0f * v);
  }
  cnorm[(size_t)h * C + ci] = s;
}

static int launch_assign_km(const void* X, const void* cen, int32_t* lab, int H, int N, int C,
                            int pin_begin, int pin_label, uint16_t* cprep, float* cnorm,
                            const int32_t* guess, hipStream_t st) {
  hipLaunchKernelGGL(cen_prep_kernel, dim3(cdiv(C, 256), H), dim3(256), 0, st,
                     (const uint16_t*)cen, cprep, cnorm, C);
  hipLaunchKernelGGL(assign_km_kernel<AK_CHUNK>, dim3(cdiv(N, AK_WAVES * 32 * AK_RB), H),
                     dim3(AK_WAVES * 64), 0, st, (const uint16_t*)X, (const uint16_t*)cprep,
                     (const float*)cnorm, lab, N, C, pin_begin, pin_label, guess);
  return t2t_check_launch("assign");
}

template <typename T>
static void launch_key_gather(const void* KU, const void* V, const int32_t* perm,
                              const int32_t* counts, const int32_t* cbase, const void* ck0,
                              float* ck2, void* V_sorted, float* vsum, float* cmax, int H, int N,
                              int C, long long svh, long long svn, hipStream_t st) {
  hipLaunchKernelGGL(key_gather_kernel<T>, dim3(cdiv(C, 4), H), dim3(256), 0, st,
                     (const uint16_t*)KU, (const uint16_t*)V, perm, counts, cbase,
                     (const uint16_t*)ck0, ck2, (uint16_t*)V_sorted, vsum, cmax, N, C, svh, svn);
}

#define KM_CHECK(x)            \
  do {                         \
    int _rc = (x);             \
    if (_rc) return _rc;       \
  } while (0)

static int kmm_impl(const void* QU, const void* KU, const void* V, int v_dtype,
                    const void* cq0, const void* ck0, int32_t* qlab, void* cq2, int32_t* klab,
                    float* ck2, int32_t* qcounts, int32_t* qperm, int32_t* kcounts,
                    int32_t* kperm, void* V_sorted, void* sumv, float* lam, int H, int N, int CQ,
                    int CK, int pin_tail, void* ws, size_t ws_bytes, long long svh,
                    long long svn, void* stream) {
  T2T_REQUIRE(QU && KU && V && cq0 && ck0 && qlab && cq2 && klab && ck2 && qcounts && qperm &&
                  kcounts && kperm && sumv && lam,
              "kmm_run: null pointer");  // V_sorted may be NULL: not written
  T2T_REQUIRE(v_dtype == T2T_F16 || v_dtype == T2T_BF16, "kmm_run: dtype %d", v_dtype);
  T2T_REQUIRE(H > 0 && N > 0, "kmm_run: H=%d N=%d", H, N);
  T2T_REQUIRE(CQ >= 1 && CQ <= KM_MAXC && CK >= 1 && CK <= KM_MAXC,
              "kmm_run: CQ=%d CK=%d must be in [1, %d]", CQ, CK, KM_MAXC);
  T2T_REQUIRE(pin_tail >= 0 && pin_tail <= N, "kmm_run: pin_tail must be in [0, N]");
  T2T_REQUIRE(svn >= 128 && svn % 8 == 0 && svh >= 0 && svh % 8 == 0,
              "kmm_run: V strides (%lld, %lld) must be multiples of 8, row stride >= 128", svh, svn);
  const KmmWs need = kmm_layout(H, N, CQ, CK, nullptr);
  if (!ws || ws_bytes < need.total) {
    t2t_set_error("kmm_run: workspace %zu < %zu bytes", ws_bytes, need.total);
    return T2T_ERR_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  KmmWs w = kmm_layout(H, N, CQ, CK, ws);
  const int nores = N + 1;  // no pinned rows
  // query pass 1
  // the label buffers' previous contents (the caller's labels of the last
  // call, or anything) are warm-start guesses: pass 1 starts from qlab, pass 2
  // from pass 1's labels, the key pass from klab
  KM_CHECK(launch_assign_km(QU, cq0, w.qlab1, H, N, CQ, nores, 0, w.cprep, w.cnorm, qlab, st));
  KM_CHECK(run_sort(w.qlab1, w.counts1, w.cbase1, w.perm1, w.chist, H, N, CQ, st));
  hipLaunchKernelGGL(fixed_mean_kernel<0>, dim3(cdiv(CQ, 4), H), dim3(256), 0, st,
                     (const uint16_t*)QU, w.perm1, w.counts1, w.cbase1, (const uint16_t*)cq0,
                     w.cq1, N, CQ);
  T2T_LAUNCH_CHECK("qmean 1");
  // query pass 2
  KM_CHECK(launch_assign_km(QU, w.cq1, qlab, H, N, CQ, nores, 0, w.cprep, w.cnorm, w.qlab1, st));
  KM_CHECK(run_sort(qlab, qcounts, w.cbaseq, qperm, w.chist, H, N, CQ, st));
  hipLaunchKernelGGL(fixed_mean_kernel<0>, dim3(cdiv(CQ, 4), H), dim3(256), 0, st,
                     (const uint16_t*)QU, qperm, qcounts, w.cbaseq, (const uint16_t*)w.cq1,
                     (uint16_t*)cq2, N, CQ);
  T2T_LAUNCH_CHECK("qmean 2");
  // key pass
  KM_CHECK(launch_assign_km(KU, ck0, klab, H, N, CK, pin_tail > 0 ? N - pin_tail : nores,
                            CK - 1, w.cprep, w.cnorm, klab, st));
  KM_CHECK(run_sort(klab, kcounts, w.cbasek, kperm, w.chist, H, N, CK, st));
  if (v_dtype == T2T_F16)
    launch_key_gather<F16T>(KU, V, kperm, kcounts, w.cbasek, ck0, ck2, V_sorted, w.vsum, w.cmax, H, N, CK,
                            svh, svn, st);
  else
    launch_key_gather<BF16T>(KU, V, kperm, kcounts, w.cbasek, ck0, ck2, V_sorted, w.vsum, w.cmax, H, N, CK,
                             svh, svn, st);
  T2T_LAUNCH_CHECK("key gather");
  launch_vstats(w.vsum, w.cmax, sumv, lam, H, CK, st);
  T2T_LAUNCH_CHECK("vstats");
  return T2T_OK;
}

extern "C" int t2t_kmm_run(const void* QU, const void* KU, const void* V, int v_dtype,
                           const void* cq0, const void* ck0, int32_t* qlab, void* cq2,
                           int32_t* klab, float* ck2, int32_t* qcounts, int32_t* qperm,
                           int32_t* kcounts, int32_t* kperm, void* V_sorted, void* sumv,
                           float* lam, int H, int N, int CQ, int CK, int pin_tail, void* ws,
                           size_t ws_bytes, void* stream) {
  return kmm_impl(QU, KU, V, v_dtype, cq0, ck0, qlab, cq2, klab, ck2, qcounts, qperm, kcounts,
                  kperm, V_sorted, sumv, lam, H, N, CQ, CK, pin_tail, ws, ws_bytes,
                  (long long)N * 128, 128, stream);
}

extern "C" int t2t_kmm_run_strided(const void* QU, const void* KU, const void* V, int v_dtype,
                                   long long v_head_stride, long long v_row_stride,
                                   const void* cq0, const void* ck0, int32_t* qlab, void* cq2,
                                   int32_t* klab, float* ck2, int32_t* qcounts, int32_t* qperm,
                                   int32_t* kcounts, int32_t* kperm, void* V_sorted, void* sumv,
                                   float* lam, int H, int N, int CQ, int CK, int pin_tail,
                                   void* ws, size_t ws_bytes, void* stream) {
  return kmm_impl(QU, KU, V, v_dtype, cq0, ck0, qlab, cq2, klab, ck2, qcounts, qperm, kcounts,
                  kperm, V_sorted, sumv, lam, H, N, CQ, CK, pin_tail, ws, ws_bytes, v_head_stride,
                  v_row_stride, stream);
}

// ---- value statistics of a reuse call ----
struct VWs {
  int32_t* cbase;
  float* vsum;
  float* cmax;
  size_t total;
};
static VWs vws_layout(int H, int CK, void* base) {
  WsCarver w(base);
  VWs v;
  v.cbase = w.take<int32_t>((size_t)H * CK);
  v.vsum = w.take<float>((size_t)H * CK * 128);
  v.cmax = w.take<float>((size_t)H * CK);
  v.total = w.off;
  return v;
}

extern "C" size_t t2t_vstats_ws_bytes(int H, int N, int CK) {
  (void)N;
  return vws_layout(H, CK, nullptr).total;
}

static int vstats_common(const void* V, int v_dtype, const int32_t* kperm, const int32_t* kcounts,
                         void* V_sorted, void* sumv, float* lam, int H, int N, int CK, void* ws,
                         size_t ws_bytes, long long svh, long long svn, hipStream_t st) {
  T2T_REQUIRE(V && kcounts && sumv && lam, "vstats: null pointer");
  T2T_REQUIRE(v_dtype == T2T_F16 || v_dtype == T2T_BF16, "vstats: dtype %d", v_dtype);
  T2T_REQUIRE(H > 0 && N > 0 && CK >= 1 && CK <= KM_MAXC, "vstats: H=%d N=%d CK=%d", H, N, CK);
  T2T_REQUIRE(svn >= 128 && svn % 8 == 0 && svh >= 0 && svh % 8 == 0,
              "vstats: V strides (%lld, %lld) must be multiples of 8, row stride >= 128", svh, svn);
  const size_t need = vws_layout(H, CK, nullptr).total;
  if (!ws || ws_bytes < need) {
    t2t_set_error("vstats: workspace %zu < %zu bytes", ws_bytes, need);
    return T2T_ERR_WORKSPACE;
  }
  VWs w = vws_layout(H, CK, ws);
  hipLaunchKernelGGL(cbase_kernel, dim3(H), dim3(1024), 0, st, kcounts, w.cbase, CK);
  if (v_dtype == T2T_F16)
    launch_key_gather<F16T>(nullptr, V, kperm, kcounts, w.cbase, nullptr, nullptr, V_sorted,
                            w.vsum, w.cmax, H, N, CK, svh, svn, st);
  else
    launch_key_gather<BF16T>(nullptr, V, kperm, kcounts, w.cbase, nullptr, nullptr, V_sorted,
                             w.vsum, w.cmax, H, N, CK, svh, svn, st);
  launch_vstats(w.vsum, w.cmax, sumv, lam, H, CK, st);
  T2T_LAUNCH_CHECK("vstats");
  return T2T_OK;
}

extern "C" int t2t_kmm_run_vstats_gather(const void* V, int v_dtype, const int32_t* kperm,
                                         const int32_t* kcounts, void* V_sorted, void* sumv,
                                         float* lam, int H, int N, int CK, void* ws,
                                         size_t ws_bytes, void* stream) {
  T2T_REQUIRE(kperm, "vstats_gather: null kperm");  // V_sorted may be NULL: not written
  return vstats_common(V, v_dtype, kperm, kcounts, V_sorted, sumv, lam, H, N, CK, ws, ws_bytes,
                       (long long)N * 128, 128, (hipStream_t)stream);
}

extern "C" int t2t_kmm_run_vstats_gather_strided(const void* V, int v_dtype,
                                                 long long v_head_stride, long long v_row_stride,
                                                 const int32_t* kperm, const int32_t* kcounts,
                                                 void* V_sorted, void* sumv, float* lam, int H,
                                                 int N, int CK, void* ws, size_t ws_bytes,
                                                 void* stream) {
  T2T_REQUIRE(kperm, "vstats_gather: null kperm");  // V_sorted may be NULL: not written
  return vstats_common(V, v_dtype, kperm, kcounts, V_sorted, sumv, lam, H, N, CK, ws, ws_bytes,
                       v_head_stride, v_row_stride, (hipStream_t)stream);
}

extern "C" int t2t_kmm_run_vstats(const void* V_sorted, int v_dtype, const int32_t* kcounts,
                                  void* sumv, float* lam, int H, int N, int CK, void* ws,
                                  size_t ws_bytes, void* stream) {
  return vstats_common(V_sorted, v_dtype, nullptr, kcounts, nullptr, sumv, lam, H, N, CK, ws,
                       ws_bytes, (long long)N * 128, 128, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// init_state helpers
// ---------------------------------------------------------------------------
extern "C" int t2t_fast_assign(const void* x, const void* c, int32_t* labels, int H, int N, int C,
                               int D, void* stream) {
  T2T_REQUIRE(x && c && labels, "fast_assign: null pointer");
  T2T_REQUIRE(H > 0 && N > 0 && C >= 1 && C <= KM_MAXC, "fast_assign: H=%d N=%d C=%d", H, N, C);
  T2T_REQUIRE(D == 32 || D == 64 || D == 128, "fast_assign: D=%d not in {32, 64, 128}", D);
  hipStream_t st = (hipStream_t)stream;
  int ibits = 1;
  while ((1 << ibits) < C) ++ibits;
  const dim3 g(cdiv(N, 128), H);
  if (D == 32)
    hipLaunchKernelGGL((fast_assign_kernel<32>), g, dim3(256), 0, st, (const uint16_t*)x,
                       (const uint16_t*)c, labels, N, C, ibits);
  else if (D == 64)
    hipLaunchKernelGGL((fast_assign_kernel<64>), g, dim3(256), 0, st, (const uint16_t*)x,
                       (const uint16_t*)c, labels, N, C, ibits);
  else
    hipLaunchKernelGGL((fast_assign_kernel<128>), g, dim3(256), 0, st, (const uint16_t*)x,
                       (const uint16_t*)c, labels, N, C, ibits);
  T2T_LAUNCH_CHECK("fast_assign");
  return T2T_OK;
}

struct DetWs {
  int32_t* perm;
  int32_t* cbase;
  int32_t* chist;
  size_t total;
};
static DetWs det_layout(int H, int N, int C, void* base) {
  WsCarver w(base);
  DetWs d;
  d.perm = w.take<int32_t>((size_t)H * N);
  d.cbase = w.take<int32_t>((size_t)H * C);
  d.chist = w.take<int32_t>((size_t)H * cdiv(N, SORT_CH) * C);
  d.total = w.off;
  return d;
}

extern "C" size_t t2t_det_update_ws_bytes(int H, int N, int C) {
  return det_layout(H, N, C, nullptr).total;
}

// ---------------------------------------------------------------------------
// fp32 centroid means and per-cluster value means (the reference's
// fused_update_vstats): one wave per cluster sums its rows in sorted order,
// fp32 and sequential per dim (lanes 0..31: one dim of x each; all lanes: two
// dims of v each).  Empty clusters: centroid = fp32(old), value mean = 0.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void seg_mean_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ V,
    const int32_t* __restrict__ perm, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ cbase, const uint16_t* __restrict__ old,
    float* __restrict__ cent, float* __restrict__ vmean, int N, int C) {
  const int h = blockIdx.y;
  const int l = threadIdx.x & 63;
  const int c = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (c >= C) return;
  const int n = counts[(size_t)h * C + c];
  const int32_t* ph = perm + (size_t)h * N + cbase[(size_t)h * C + c];
  const uint16_t* xh = X + (size_t)h * N * KM_R;
  const uint32_t* vh = V ? (const uint32_t*)(V + (size_t)h * N * 128) : nullptr;
  float ax = 0.f, v0 = 0.f, v1 = 0.f;
  for (int i0 = 0; i0 < n; i0 += 64) {
    const int myrow = i0 + l < n ? ph[i0 + l] : 0;
    const int m = n - i0 < 64 ? n - i0 : 64;
    for (int i = 0; i < m; ++i) {
      const int rw = __builtin_amdgcn_readlane(myrow, i);
      if (l < KM_R) ax += h2f(xh[(size_t)rw * KM_R + l]);
      if (vh) {
        const uint32_t u = vh[(size_t)rw * 64 + l];
        v0 += T::to_f((uint16_t)(u & 0xffff));
        v1 += T::to_f((uint16_t)(u >> 16));
      }
    }
  }
  if (l < KM_R) {
    const size_t o = ((size_t)h * C + c) * KM_R + l;
    cent[o] = n ? ax / (float)n : h2f(old[o]);
  }
  if (vh) {
    const float d = n ? (float)n : 1.0f;
    float* vo = vmean + ((size_t)h * C + c) * 128 + 2 * l;
    vo[0] = v0 / d;
    vo[1] = v1 / d;
  }
}

extern "C" int t2t_fused_update_vstats(const void* x, const int32_t* labels, const void* old,
                                       const void* v, int v_dtype, float* cent, int32_t* counts,
                                       float* vmean, int H, int N, int C, int D, void* ws,
                                       size_t ws_bytes, void* stream) {
  T2T_REQUIRE(x && labels && old && cent && counts, "fused_update_vstats: null pointer");
  T2T_REQUIRE(!v || vmean, "fused_update_vstats: v given without vmean");
  T2T_REQUIRE(!v || v_dtype == T2T_F16 || v_dtype == T2T_BF16, "fused_update_vstats: dtype %d",
              v_dtype);
  T2T_REQUIRE(H > 0 && N > 0 && C >= 1 && C <= KM_MAXC, "fused_update_vstats: H=%d N=%d C=%d", H,
              N, C);
  T2T_REQUIRE(D == KM_R, "fused_update_vstats: D=%d (built for %d)", D, KM_R);
  const size_t need = det_layout(H, N, C, nullptr).total;
  if (!ws || ws_bytes < need) {
    t2t_set_error("fused_update_vstats: workspace %zu < %zu bytes", ws_bytes, need);
    return T2T_ERR_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  DetWs w = det_layout(H, N, C, ws);
  KM_CHECK(run_sort(labels, counts, w.cbase, w.perm, w.chist, H, N, C, st));
  const dim3 g(cdiv(C, 4), H);
  if (v && v_dtype == T2T_BF16)
    hipLaunchKernelGGL(seg_mean_kernel<BF16T>, g, dim3(256), 0, st, (const uint16_t*)x,
                       (const uint16_t*)v, w.perm, counts, w.cbase, (const uint16_t*)old, cent,
                       vmean, N, C);
  else
    hipLaunchKernelGGL(seg_mean_kernel<F16T>, g, dim3(256), 0, st, (const uint16_t*)x,
                       (const uint16_t*)v, w.perm, counts, w.cbase, (const uint16_t*)old, cent,
                       vmean, N, C);
  T2T_LAUNCH_CHECK("fused_update_vstats");
  return T2T_OK;
}

extern "C" int t2t_det_centroid_update(const void* x, const int32_t* labels, const void* old,
                                       void* out, int32_t* counts, int H, int N, int C, int D,
                                       void* ws, size_t ws_bytes, void* stream) {
  T2T_REQUIRE(x && labels && old && out && counts, "det_update: null pointer");
  T2T_REQUIRE(H > 0 && N > 0 && C >= 1 && C <= KM_MAXC, "det_update: H=%d N=%d C=%d", H, N, C);
  T2T_REQUIRE(D == KM_R, "det_update: D=%d (built for %d)", D, KM_R);
  const size_t need = det_layout(H, N, C, nullptr).total;
  if (!ws || ws_bytes < need) {
    t2t_set_error("det_update: workspace %zu < %zu bytes", ws_bytes, need);
    return T2T_ERR_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  DetWs w = det_layout(H, N, C, ws);
  KM_CHECK(run_sort(labels, counts, w.cbase, w.perm, w.chist, H, N, C, st));
  hipLaunchKernelGGL(fixed_mean_kernel<1>, dim3(cdiv(C, 4), H), dim3(256), 0, st,
                     (const uint16_t*)x, w.perm, counts, w.cbase, (const uint16_t*)old,
                     (uint16_t*)out, N, C);
  T2T_LAUNCH_CHECK("det_update");
  return T2T_OK;
}
