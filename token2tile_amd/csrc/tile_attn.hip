// S5/S6: task planning, exact attention over each query cluster's union of
// key clusters, and the centroid residual + merge (gfx950, MFMA 32x32x16).
//
// Exact attention (one work-group per task of <= 256 sorted queries of one
// query cluster, 8 waves x 32 queries):
//   * the union is turned into runs of cluster-ordered key rows in LDS;
//   * 64-key tiles of K (row major) and V (transposed, key-contiguous) are
//     gathered from kp/vp into a double-buffered LDS ring: tile t is consumed
//     while tile t+1 is written from registers and tile t+2 is in flight, one
//     barrier per tile;
//   * the running max advances with a margin, so O is rescaled only when a
//     tile raises the max by more than the margin;
//   * S^T = K Q^T and O^T = V^T P^T on MFMA, so every lane owns one query:
//     the online-softmax max/sum need one cross-half exchange, and the
//     per-query rescale of O touches only the lane's own registers.
// Residual (one work-group per 128 sorted queries): the same structure over
// the 2048 centroids (K = cks, V = sumv), masked by the query's union,
// followed by the merge with the exact part.
#include "t2t_common.h"
#include <type_traits>

#define TA_D 128
#define TA_CK 2048
#define TA_QT 128   // queries per task (4 waves x 32)
#define TA_WAVES 4
#define TA_KT 64    // keys per tile
#define TA_VP 68    // residual-only sVt pitch (halves) of the unfused tail kernel

// ---------------------------------------------------------------------------
// plan layout (int32): k_off [H][2049] | kvlen [H][CQ] | ntask [H] |
//                      tasks [H][maxT][4] = (cluster, sorted start, rows, 0)
// ---------------------------------------------------------------------------
static inline int plan_max_tasks(int N, int CQ) { return CQ + cdiv(N, TA_QT) + 1; }

struct PlanView {
  int32_t* k_off;
  int32_t* kvlen;
  int32_t* ntask;
  int32_t* tasks;
  int maxT;
};
static PlanView plan_view(int32_t* plan, int H, int N, int CQ) {
  PlanView p;
  p.maxT = plan_max_tasks(N, CQ);
  p.k_off = plan;
  p.kvlen = p.k_off + (size_t)H * (TA_CK + 1);
  p.ntask = p.kvlen + (size_t)H * CQ;
  p.tasks = p.ntask + H;
  return p;
}

extern "C" size_t t2t_tile_plan_ints(int H, int N, int CQ) {
  return (size_t)H * (TA_CK + 1) + (size_t)H * CQ + H + (size_t)H * plan_max_tasks(N, CQ) * 4;
}

#define PLAN_SORT_MAX 4096

__global__ __launch_bounds__(1024) void plan_kernel(const int32_t* __restrict__ qcounts,
                                                    const int32_t* __restrict__ kcounts,
                                                    const uint32_t* __restrict__ unip,
                                                    int32_t* __restrict__ k_off,
                                                    int32_t* __restrict__ kvlen,
                                                    int32_t* __restrict__ ntask,
                                                    int32_t* __restrict__ tasks, int CQ, int maxT) {
  __shared__ int sk[TA_CK];
  __shared__ int wsum[16];
  __shared__ int carry;
  __shared__ unsigned long long skey[PLAN_SORT_MAX];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // key-cluster offsets (2 clusters per thread, in order)
  const int c0 = 2 * tid;
  const int a0 = kcounts[(size_t)h * TA_CK + c0], a1 = kcounts[(size_t)h * TA_CK + c0 + 1];
  sk[c0] = a0;
  sk[c0 + 1] = a1;
  int inc = wave_incl_scan(a0 + a1);
  if (lane == 63) wsum[w] = inc;
  __syncthreads();
  int ex = inc - a0 - a1;
  for (int i = 0; i < w; ++i) ex += wsum[i];
  int32_t* ko = k_off + (size_t)h * (TA_CK + 1);
  ko[c0] = ex;
  ko[c0 + 1] = ex + a0;
  if (tid == 1023) ko[TA_CK] = ex + a0 + a1;
  __syncthreads();
  // union lengths: one wave per query cluster
  for (int t = w; t < CQ; t += 16) {
    int s = 0;
    if (qcounts[(size_t)h * CQ + t] > 0) {
      uint32_t bits = unip[((size_t)h * CQ + t) * (TA_CK / 32) + lane];
      while (bits) {
        const int b = __builtin_ctz(bits);
        s += sk[lane * 32 + b];
        bits &= bits - 1;
      }
    }
    s = wave_sum(s);
    if (lane == 0) kvlen[(size_t)h * CQ + t] = s;
  }
  __syncthreads();
  // task list: cluster t splits into ceil(n / QT) balanced tasks
  if (tid == 0) carry = 0;
  __syncthreads();
  __shared__ int qcarry;
  if (tid == 0) qcarry = 0;
  __syncthreads();
  int32_t* th = tasks + (size_t)h * maxT * 4;
  for (int b0 = 0; b0 < CQ; b0 += 1024) {
    const int t = b0 + tid;
    const int n = t < CQ ? qcounts[(size_t)h * CQ + t] : 0;
    const int nt = (n + TA_QT - 1) / TA_QT;
    int ti = wave_incl_scan(nt);
    int qi = wave_incl_scan(n);
    __syncthreads();
    if (lane == 63) wsum[w] = ti;
    __syncthreads();
    int tex = ti - nt + carry;
    for (int i = 0; i < w; ++i) tex += wsum[i];
    const int tot_t = [&] { int s = 0; for (int i = 0; i < 16; ++i) s += wsum[i]; return s; }();
    __syncthreads();
    if (lane == 63) wsum[w] = qi;
    __syncthreads();
    int qex = qi - n + qcarry;
    for (int i = 0; i < w; ++i) qex += wsum[i];
    const int tot_q = [&] { int s = 0; for (int i = 0; i < 16; ++i) s += wsum[i]; return s; }();
    if (t < CQ && nt > 0) {
      const int base = n / nt, rem = n % nt;
      int s = qex;
      for (int i = 0; i < nt; ++i) {
        const int rows = base + (i < rem ? 1 : 0);
        int32_t* tk = th + (size_t)(tex + i) * 4;
        tk[0] = t;
        tk[1] = s;
        tk[2] = rows;
        tk[3] = 0;
        s += rows;
      }
    }
    __syncthreads();
    if (tid == 0) {
      carry += tot_t;
      qcarry += tot_q;
    }
    __syncthreads();
  }
  const int nT = carry;
  if (tid == 0) ntask[h] = nT;
  __syncthreads();
  if (nT > PLAN_SORT_MAX || nT < 2) return;
  // LPT order: descending rows x kv_len, ties by lower task index
  int P2 = 2;
  while (P2 < nT) P2 <<= 1;
  for (int i = tid; i < P2; i += 1024) {
    unsigned long long key = 0ull;
    if (i < nT) {
      const int32_t* tk = th + (size_t)i * 4;
      unsigned long long work =
          (unsigned long long)tk[2] * (unsigned long long)kvlen[(size_t)h * CQ + tk[0]];
      if (work > 0xFFFFFFFFull) work = 0xFFFFFFFFull;
      key = (work << 32) | (unsigned long long)(0x7FFFFFFF - i);
    }
    skey[i] = key;
  }
  __syncthreads();
  for (int k = 2; k <= P2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < P2; i += 1024) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const unsigned long long x = skey[i], y = skey[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) {
            skey[i] = y;
            skey[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  // permute in place through registers (<= 4 tasks per thread)
  int4 mine[PLAN_SORT_MAX / 1024];
  int nm = 0;
  for (int i = tid; i < nT; i += 1024) {
    const int src = 0x7FFFFFFF - (int)(skey[i] & 0xFFFFFFFFull);
    mine[nm++] = *(const int4*)(th + (size_t)src * 4);
  }
  __syncthreads();
  nm = 0;
  for (int i = tid; i < nT; i += 1024) *(int4*)(th + (size_t)i * 4) = mine[nm++];
}

extern "C" int t2t_tile_plan(const int32_t* qcounts, const int32_t* kcounts, const int32_t* unip,
                             int32_t* plan, int H, int N, int CQ, void* stream) {
  T2T_REQUIRE(qcounts && kcounts && unip && plan, "tile_plan: null pointer");
  T2T_REQUIRE(H > 0 && N > 0 && CQ > 0, "tile_plan: H=%d N=%d CQ=%d", H, N, CQ);
  PlanView p = plan_view(plan, H, N, CQ);
  hipLaunchKernelGGL(plan_kernel, dim3(H), dim3(1024), 0, (hipStream_t)stream, qcounts, kcounts,
                     (const uint32_t*)unip, p.k_off, p.kvlen, p.ntask, p.tasks, CQ, p.maxT);
  T2T_LAUNCH_CHECK("tile_plan");
  return T2T_OK;
}

// ---------------------------------------------------------------------------
// exact attention
// ---------------------------------------------------------------------------
__device__ inline uint32_t pack2(uint16_t a, uint16_t b) { return (uint32_t)a | ((uint32_t)b << 16); }

// map a linear block id to a task so that each XCD (8 of them, blocks are
// dealt round-robin) works through a contiguous range of the task list
__device__ inline int xcd_remap(int bid, int total) {
  const int per = (total + 7) / 8;
  return (bid % 8) * per + bid / 8;
}

#define TA_MARGIN 3.0f   // log2 units of headroom when the exact-part max advances
#define TL_MARGIN 2.0f   // natural-log units of headroom for the residual max
#define TL_CT 64         // centroids per residual tile
#define TL_CP 40         // residual centroid tile pitch (halves)

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// LDS tile layouts (no padding, XOR swizzles keep the MFMA operand reads
// conflict free):
//   sK  [64 keys][128 dims]: 16-byte chunk c of row r lives at chunk c ^ (r & 15)
//   sVt [128 dims][64 keys]: the 4-key granules a lane feeds to one MFMA
//     (g = 4 m + h and 4 m + 2 + h) are stored side by side, so the operand is
//     one 16-byte read: granule g sits in 16-byte unit (g & ~3) / 2 + (g & 1),
//     half (g >> 1) & 1, and the unit is XOR-swizzled by ((d >> 1) ^ (d >> 4)) & 7
__device__ inline int sk_off(int row, int chunk) { return row * 128 + 8 * (chunk ^ (row & 15)); }
__device__ inline int vt_swz(int dim) { return ((dim >> 1) ^ (dim >> 4)) & 7; }
__device__ inline int vt_unit_off(int dim, int unit) { return dim * 64 + 8 * (unit ^ vt_swz(dim)); }
__device__ inline int vt_gran_off(int dim, int g) {
  return vt_unit_off(dim, ((g & ~3) >> 1) + (g & 1)) + 4 * ((g >> 1) & 1);
}

__device__ inline float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
// (b.lo16 << 16) | a.lo16 and (b.hi16 << 16) | a.hi16
__device__ inline uint32_t pack_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ inline uint32_t pack_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }
// keeps the compiler from if-converting a rarely taken block into selects
#define T2T_REAL_BRANCH() asm volatile("" ::: "memory")

// One work-group (4 waves, 32 queries each) per task of <= 128 queries, two
// work-groups per CU.  FUSE = false: exact attention only, attn_out and lse
// (log2 units) in sorted order.  FUSE = true: exact attention, then the
// residual over the centroids outside the task's (shared) union and the
// merge under one softmax, written at the original rows.
template <typename T, bool FUSE>
__global__ __launch_bounds__(TA_WAVES * 64, 2) void attn_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kp,
    const uint16_t* __restrict__ vp, const uint32_t* __restrict__ unip,
    const int32_t* __restrict__ qperm, const int32_t* __restrict__ kcounts,
    const int32_t* __restrict__ k_off, const int32_t* __restrict__ ntask,
    const int32_t* __restrict__ tasks, uint16_t* __restrict__ attn_out, float* __restrict__ lse,
    const uint16_t* __restrict__ QU, const uint16_t* __restrict__ cks,
    const uint16_t* __restrict__ sumv, const float* __restrict__ lam,
    const float* __restrict__ tailw, uint16_t* __restrict__ out, int H, int N, int CQ, int maxT) {
  __shared__ __attribute__((aligned(1024))) uint16_t sK[2][TA_KT * 128];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[2][TA_D * 64];
  __shared__ uint16_t runCl[TA_CK];
  __shared__ int runCum[TA_CK + 1];
  __shared__ int sIdx[2][TA_KT];
  __shared__ __attribute__((aligned(16))) float sCnt[2][TL_CT];
  __shared__ int wsc[TA_WAVES], wsr[TA_WAVES];
  const int total = H * maxT;
  const int lin = xcd_remap(blockIdx.x, total);
  if (lin >= total) return;
  const int h = lin / maxT, ti = lin % maxT;
  if (ti >= ntask[h]) return;
  const int32_t* tk = tasks + ((size_t)h * maxT + ti) * 4;
  const int t = tk[0], qs = tk[1], qrows = tk[2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int jl = lane & 31, hh = lane >> 5;

  // ---- runs of selected, non-empty key clusters (ascending cluster order);
  //      thread tid owns clusters 8 tid .. 8 tid + 7
  const uint32_t* ur = unip + ((size_t)h * CQ + t) * (TA_CK / 32);
  const int32_t* ko = k_off + (size_t)h * (TA_CK + 1);
  const int32_t* kc = kcounts + (size_t)h * TA_CK;
  const uint32_t byte = (ur[tid >> 2] >> (8 * (tid & 3))) & 0xffu;
  int cnts[8];
  int nr = 0, ns = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    cnts[j] = ((byte >> j) & 1u) ? kc[8 * tid + j] : 0;
    nr += cnts[j] > 0;
    ns += cnts[j];
  }
  const int ir = wave_incl_scan(nr), is = wave_incl_scan(ns);
  if (lane == 63) {
    wsc[wave] = ir;
    wsr[wave] = is;
  }
  __syncthreads();
  int r = ir - nr, p = is - ns, nrun = 0, kvlen = 0;
#pragma unroll
  for (int i = 0; i < TA_WAVES; ++i) {
    if (i < wave) {
      r += wsc[i];
      p += wsr[i];
    }
    nrun += wsc[i];
    kvlen += wsr[i];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (cnts[j] > 0) {
      runCl[r] = (uint16_t)(8 * tid + j);
      runCum[r] = p;
      ++r;
      p += cnts[j];
    }
  }
  if (tid == 0) runCum[nrun] = kvlen;

  const int qrow = wave * 32 + jl;  // query row inside the task
  const bool qok = qrow < qrows;
  const bool wave_active = wave * 32 < qrows;
  const size_t obase = (size_t)h * N + qs;  // sorted-order rows of the task
  const int orig = qperm[obase + (qok ? qrow : 0)];
  const int kq = tid >> 4, dseg = tid & 15;  // V loader: 4 keys (4 kq ..) x 8 dims (dseg)

  // ---- stage 4 rows x 8 dims into the transposed, swizzled sVt[buf]
  auto stash_vt = [&](int buf, const u32x4 (&v)[4]) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const u32x2 lo = {pack_lo(v[0][w], v[1][w]), pack_lo(v[2][w], v[3][w])};
      const u32x2 hi = {pack_hi(v[0][w], v[1][w]), pack_hi(v[2][w], v[3][w])};
      *(u32x2*)(sVt[buf] + vt_gran_off(8 * dseg + 2 * w, kq)) = lo;
      *(u32x2*)(sVt[buf] + vt_gran_off(8 * dseg + 2 * w + 1, kq)) = hi;
    }
  };
  // ---- O^T += V^T P^T over one 64-key tile
  auto pv = [&](f32x16 (&Oa)[4], int buf, const u32x4 (&pb)[4], auto mf) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int dim = 32 * nb + jl;
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        const u32x4 a = *(const u32x4*)(sVt[buf] + vt_unit_off(dim, 2 * mm + hh));
        Oa[nb] = mf(a, pb[mm], Oa[nb]);
      }
    }
  };
  auto rescale = [&](f32x16 (&Oa)[4], float alpha) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int a = 0; a < 16; ++a) Oa[nb][a] *= alpha;
  };

  const float c = 0.08838834764831845f * 1.4426950408889634f;  // 1/sqrt(128) * log2(e)
  float m = -__builtin_inff(), lsum = 0.f;
  f32x16 O[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) O[nb] = zero16();

  if (kvlen > 0) {
    // ---- queries: B operand fragments (dims 16 s + 8 hh .. + 7)
    u32x4 qb[8];
    {
      const uint16_t* qr = q + ((size_t)h * N + orig) * TA_D + 8 * hh;
#pragma unroll
      for (int s = 0; s < 8; ++s) qb[s] = *(const u32x4*)(qr + 16 * s);
    }
    const char* kh = (const char*)(kp + (size_t)h * N * TA_D);
    const char* vh = (const char*)(vp + (size_t)h * N * TA_D) + 16 * dseg;
    const int ntile = (kvlen + TA_KT - 1) / TA_KT;
    int cur = 0;  // run cursor of the index builders (threads 0..63)
    // source rows of tile `tile` -> sIdx[tile & 1]; past the end -> row 0
    // (its keys are masked and its values multiply a zero probability)
    auto build_idx = [&](int tile) {
      if (tid < TA_KT) {
        const int pos = tile * TA_KT + tid;
        int row = 0;
        if (pos < kvlen) {
          while (runCum[cur + 1] <= pos) ++cur;
          row = ko[runCl[cur]] + pos - runCum[cur];
        }
        sIdx[tile & 1][tid] = row;
      }
    };
    u32x4 ldv[4];
    // K tile via LDS DMA (each wave instruction fills 4 whole rows, the lane
    // fetching the chunk that belongs at its swizzled position), V tile into
    // registers for the transposed store
    auto issue = [&](int tile) {
      const int buf = tile & 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int blk = 4 * i + wave;
        const int row = 4 * blk + (lane >> 4);
        const uint32_t off = (uint32_t)sIdx[buf][row] * 256u + 16u * ((lane & 15) ^ (row & 15));
        __builtin_amdgcn_global_load_lds((const glb_void_t*)(kh + off),
                                         (lds_void_t*)(sK[buf] + blk * 4 * 128), 16, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ldv[i] = *(const u32x4*)(vh + (uint32_t)sIdx[buf][4 * kq + i] * 256u);
    };
    // one 64-key tile of the online softmax; MASK: the last, partial tile
    auto tile_step = [&](int buf, int valid, auto MASK) {
      f32x16 S[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        S[kb] = zero16();
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const u32x4 a = *(const u32x4*)(sK[buf] + sk_off(32 * kb + jl, 2 * s + hh));
          S[kb] = Mfma<T>::run(a, qb[s], S[kb]);
        }
      }
      if constexpr (decltype(MASK)::value) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int a = 0; a < 16; ++a)
            if (32 * kb + 8 * (a / 4) + 4 * hh + (a % 4) >= valid) S[kb][a] = -__builtin_inff();
      }
      float mr = -__builtin_inff();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int a = 0; a < 16; a += 2) mr = vmax(mr, vmax(S[kb][a], S[kb][a + 1]));
      mr = vmax(mr, __shfl_xor(mr, 32, 64));
      const float mx = mr * c;
      // lazy max: move only when exceeded, then with headroom
      if (__builtin_amdgcn_readfirstlane((int)(__ballot(mx > m) != 0ull))) {
        T2T_REAL_BRANCH();
        const float mnew = mx > m ? mx + TA_MARGIN : m;
        const float alpha = __builtin_amdgcn_exp2f(m - mnew);
        m = mnew;
        lsum *= alpha;
        rescale(O, alpha);
      }
      const float nm = -m;
      u32x4 pb[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int a = 0; a < 16; a += 2) {
          const float p0 = __builtin_amdgcn_exp2f(fmaf(S[kb][a], c, nm));
          const float p1 = __builtin_amdgcn_exp2f(fmaf(S[kb][a + 1], c, nm));
          const uint32_t pk = Pk<T>::pack(p0, p1);
          lsum = Pk<T>::sum2(pk, lsum);
          pb[2 * kb + a / 8][(a % 8) / 2] = pk;
        }
      pv(O, buf, pb, [](const u32x4& a_, const u32x4& b_, const f32x16& c_) {
        return Mfma<T>::run(a_, b_, c_);
      });
    };
    __syncthreads();  // runs visible
    build_idx(0);
    if (ntile > 1) build_idx(1);
    __syncthreads();
    issue(0);
    stash_vt(0, ldv);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (ntile > 1) issue(1);
    if (ntile > 2) build_idx(2);
    // full tiles in the loop; a partial last tile is peeled after it (one
    // masked copy of the tile body outside the loop keeps register pressure
    // of the loop at that of the unmasked body)
    const int nfull = (kvlen % TA_KT) ? ntile - 1 : ntile;
    int tile = 0;
    for (; tile < nfull; ++tile) {
      const int buf = tile & 1;
      if (wave_active) tile_step(buf, TA_KT, std::false_type{});
      if (tile + 1 < ntile) stash_vt(buf ^ 1, ldv);
      __builtin_amdgcn_s_waitcnt(0);  // K DMA of tile + 1 landed
      __syncthreads();
      if (tile + 2 < ntile) issue(tile + 2);
      if (tile + 3 < ntile) build_idx(tile + 3);
    }
    if (tile < ntile && wave_active) tile_step(tile & 1, kvlen - tile * TA_KT, std::true_type{});
  }
  const float lt = lsum + __shfl_xor(lsum, 32, 64);
  const float inv = kvlen > 0 ? 1.0f / lt : 0.f;
  const float lse2 = kvlen > 0 ? m + __log2f(lt) : -__builtin_inff();
  // exact output of the lane's 64 dims, rounded to T as the exact buffer
  // holds it: sorted-order attn_out (exact-only kernel) or, for the fused
  // kernel, the original row of out, read back by the merge
  if (qok) {
    uint16_t* orow = FUSE ? out + ((size_t)h * N + orig) * TA_D : attn_out + (obase + qrow) * TA_D;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(u32x2*)(orow + 32 * nb + 8 * g + 4 * hh) =
            u32x2{Pk<T>::pack(O[nb][4 * g] * inv, O[nb][4 * g + 1] * inv),
                  Pk<T>::pack(O[nb][4 * g + 2] * inv, O[nb][4 * g + 3] * inv)};
  }
  if constexpr (!FUSE) {
    if (qok && hh == 0) lse[obase + qrow] = lse2;
    return;
  } else {
    // ---------------- residual over the centroids outside the union ----------
    // Centroids inside the union are staged with zero count and zero value
    // sum, so they add nothing to phi or O and need no per-score test.
    const float L2E = 1.4426950408889634f;
    uint32_t todo = 0;  // centroid tiles not entirely inside the union
#pragma unroll 1
    for (int tc = 0; tc < TA_CK / TL_CT; ++tc)
      if ((ur[2 * tc] & ur[2 * tc + 1]) != 0xffffffffu) todo |= 1u << tc;
    u32x4 qu0, qu1;
    {
      const uint16_t* qr = QU + ((size_t)h * N + orig) * 32 + 8 * hh;
      qu0 = *(const u32x4*)(qr);
      qu1 = *(const u32x4*)(qr + 16);
    }
    const uint16_t* chh = cks + (size_t)h * TA_CK * 32;
    const uint16_t* shh = sumv + (size_t)h * TA_CK * TA_D + 8 * dseg;
    u32x4 lc, lv[4];
    float lcnt = 0.f;
    auto issue_r = [&](int tc) {
      lc = *(const u32x4*)(chh + (size_t)(tc * TL_CT + (tid >> 2)) * 32 + 8 * (tid & 3));
      const uint32_t w4 = (ur[2 * tc + (kq >> 3)] >> (4 * (kq & 7))) & 0xfu;  // my 4 centroids
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lv[i] = *(const u32x4*)(shh + (size_t)(tc * TL_CT + 4 * kq + i) * TA_D);
        if ((w4 >> i) & 1u) lv[i] = u32x4{0u, 0u, 0u, 0u};
      }
      if (tid < TL_CT)
        lcnt = ((ur[2 * tc + (tid >> 5)] >> (tid & 31)) & 1u) ? 0.f : (float)kc[tc * TL_CT + tid];
    };
    auto stash_r = [&](int buf) {
      *(u32x4*)(sK[buf] + (tid >> 2) * TL_CP + 8 * (tid & 3)) = lc;
      stash_vt(buf, lv);
      if (tid < TL_CT) sCnt[buf][tid] = lcnt;
    };
    float m2 = -__builtin_inff(), phi = 0.f;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) O[nb] = zero16();
    __syncthreads();  // the exact loop's buffers are free
    uint32_t rest = todo;
    int tcur = rest ? __builtin_ctz(rest) : -1;
    if (rest) rest &= rest - 1;
    int tnext = rest ? __builtin_ctz(rest) : -1;
    if (rest) rest &= rest - 1;
    if (tcur >= 0) {
      issue_r(tcur);
      stash_r(0);
      if (tnext >= 0) issue_r(tnext);
    }
    __syncthreads();
    int buf = 0;
    while (tcur >= 0) {
      // scores of the lane's query against 32 kb + 8 (a / 4) + 4 hh + a % 4,
      // rounded to fp16 as the selection's scores are
      uint32_t sh[2][8];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const uint16_t* crow = sK[buf] + (32 * kb + jl) * TL_CP + 8 * hh;
        f32x16 S = zero16();
        S = Mfma<F16T>::run(*(const u32x4*)(crow), qu0, S);
        S = Mfma<F16T>::run(*(const u32x4*)(crow + 16), qu1, S);
#pragma unroll
        for (int a = 0; a < 16; a += 2) sh[kb][a / 2] = Pk<F16T>::pack(S[a], S[a + 1]);
      }
      float sv[2][16];
      float mx = -__builtin_inff();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int a = 0; a < 16; a += 2) {
          sv[kb][a] = h2f((uint16_t)(sh[kb][a / 2] & 0xffffu));
          sv[kb][a + 1] = h2f((uint16_t)(sh[kb][a / 2] >> 16));
          mx = vmax(mx, vmax(sv[kb][a], sv[kb][a + 1]));
        }
      mx = vmax(mx, __shfl_xor(mx, 32, 64));
      if (__builtin_amdgcn_readfirstlane((int)(__ballot(mx > m2) != 0ull))) {
        T2T_REAL_BRANCH();
        const float mnew = mx > m2 ? mx + TL_MARGIN : m2;
        const float alpha = __builtin_amdgcn_exp2f((m2 - mnew) * L2E);
        m2 = mnew;
        phi *= alpha;
        rescale(O, alpha);
      }
      const float nm = -m2 * L2E;
      u32x4 pb[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // counts of centroids 32 kb + 8 j + 4 hh .. + 3
          const f32x4 cn = *(const f32x4*)(sCnt[buf] + 32 * kb + 8 * j + 4 * hh);
          float pe[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pe[e] = __builtin_amdgcn_exp2f(fmaf(sv[kb][4 * j + e], L2E, nm));
            phi = fmaf(pe[e], cn[e], phi);
          }
          pb[2 * kb + j / 2][2 * (j % 2)] = Pk<F16T>::pack(pe[0], pe[1]);
          pb[2 * kb + j / 2][2 * (j % 2) + 1] = Pk<F16T>::pack(pe[2], pe[3]);
        }
      pv(O, buf, pb, [](const u32x4& a_, const u32x4& b_, const f32x16& c_) {
        return Mfma<F16T>::run(a_, b_, c_);
      });
      if (tnext >= 0) stash_r(buf ^ 1);
      const int tn2 = rest ? __builtin_ctz(rest) : -1;
      if (rest) rest &= rest - 1;
      __syncthreads();
      if (tn2 >= 0) issue_r(tn2);
      tcur = tnext;
      tnext = tn2;
      buf ^= 1;
    }
    if (!qok) return;
    // ---------------- merge under one softmax --------------------------------
    phi += __shfl_xor(phi, 32, 64);
    const float tw = *tailw;
    const float lm = lam[h];
    const float le = lse2 * 0.6931471805599453f;
    float ex, st;
    if (le >= m2) {
      ex = 1.0f;
      st = __expf(m2 - le);
    } else {
      ex = __expf(le - m2);
      st = 1.0f;
    }
    const float ph = st * phi;
    const bool bad = ph <= 1.0e-6f * ex;
    const float den = fmaxf(ex + ph * tw, 1.0e-12f);
    const float wx = ex / den, wt = st * tw * lm / den;
    if (bad) return;  // the exact part already written is the output
    uint16_t* orow = out + ((size_t)h * N + orig) * TA_D;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 v = *(const u32x2*)(orow + 32 * nb + 8 * g + 4 * hh);  // exact part
        const uint32_t w0 = v[0], w1 = v[1];
        const float x0 = T::to_f((uint16_t)(w0 & 0xffff)), x1 = T::to_f((uint16_t)(w0 >> 16));
        const float x2 = T::to_f((uint16_t)(w1 & 0xffff)), x3 = T::to_f((uint16_t)(w1 >> 16));
        v[0] = Pk<T>::pack(fmaf(wt, O[nb][4 * g], wx * x0), fmaf(wt, O[nb][4 * g + 1], wx * x1));
        v[1] = Pk<T>::pack(fmaf(wt, O[nb][4 * g + 2], wx * x2), fmaf(wt, O[nb][4 * g + 3], wx * x3));
        *(u32x2*)(orow + 32 * nb + 8 * g + 4 * hh) = v;
      }
  }
}

template <typename T, bool FUSE>
static void launch_attn(const void* q, const void* kp, const void* vp, const int32_t* unip,
                        const int32_t* qperm, const int32_t* kcounts, const PlanView& p,
                        void* attn_out, float* lse, const void* QU, const void* cks,
                        const void* sumv, const float* lam, const float* tailw, void* out, int H,
                        int N, int CQ, hipStream_t st) {
  const int total = H * p.maxT;
  const int grid = ((total + 7) / 8) * 8;
  hipLaunchKernelGGL((attn_kernel<T, FUSE>), dim3(grid), dim3(TA_WAVES * 64), 0, st,
                     (const uint16_t*)q, (const uint16_t*)kp, (const uint16_t*)vp,
                     (const uint32_t*)unip, qperm, kcounts, p.k_off, p.ntask, p.tasks,
                     (uint16_t*)attn_out, lse, (const uint16_t*)QU, (const uint16_t*)cks,
                     (const uint16_t*)sumv, lam, tailw, (uint16_t*)out, H, N, CQ, p.maxT);
}

// ---------------------------------------------------------------------------
// residual over unselected centroids + merge
// ---------------------------------------------------------------------------
#define TL_CT 64
#define TL_CP 40  // cks tile pitch (halves)

template <typename T>
__global__ __launch_bounds__(256) void tail_kernel(
    const uint16_t* __restrict__ attn_out, const float* __restrict__ attn_lse,
    const uint16_t* __restrict__ QU, const uint16_t* __restrict__ cks,
    const uint16_t* __restrict__ sumv, const int32_t* __restrict__ kcounts,
    const uint32_t* __restrict__ unip, const int32_t* __restrict__ qlab,
    const int32_t* __restrict__ qperm, const float* __restrict__ lam,
    const float* __restrict__ tailw, uint16_t* __restrict__ out, int N, int CQ) {
  __shared__ __attribute__((aligned(16))) uint16_t sC[TL_CT * TL_CP];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[TA_D * TA_VP];
  __shared__ float sCnt[TL_CT];
  const int h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int jl = lane & 31, hh = lane >> 5;
  const int j = blockIdx.x * 128 + wave * 32 + jl;  // sorted query position
  const bool ok = j < N;
  const int orig = qperm[(size_t)h * N + (ok ? j : 0)];
  const uint32_t* ur = unip + ((size_t)h * CQ + qlab[(size_t)h * N + orig]) * (TA_CK / 32);
  u32x4 qb0, qb1;
  {
    const uint16_t* qr = QU + ((size_t)h * N + orig) * 32 + 8 * hh;
    qb0 = *(const u32x4*)(qr);
    qb1 = *(const u32x4*)(qr + 16);
  }
  const uint16_t* ch = cks + (size_t)h * TA_CK * 32;
  const uint16_t* vh = sumv + (size_t)h * TA_CK * TA_D;
  const int kq = tid >> 4, dseg = tid & 15;
  const float L2E = 1.4426950408889634f;
  float m = -__builtin_inff(), phi = 0.f;
  f32x16 O[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) O[nb] = zero16();
  for (int tc = 0; tc < TA_CK / TL_CT; ++tc) {
    __syncthreads();
    {  // cks tile: 64 x 32 halves = 256 x 16 B
      const int cr = tid >> 2, cc = tid & 3;
      *(u32x4*)(sC + cr * TL_CP + 8 * cc) =
          *(const u32x4*)(ch + (size_t)(tc * TL_CT + cr) * 32 + 8 * cc);
    }
    {  // sumv tile transposed: thread = 4 centroids x 8 dims
      u32x4 v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[i] = *(const u32x4*)(vh + (size_t)(tc * TL_CT + 4 * kq + i) * TA_D + 8 * dseg);
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const int w = d >> 1, sh = (d & 1) * 16;
        u32x2 o;
        o[0] = ((v[0][w] >> sh) & 0xffffu) | (((v[1][w] >> sh) & 0xffffu) << 16);
        o[1] = ((v[2][w] >> sh) & 0xffffu) | (((v[3][w] >> sh) & 0xffffu) << 16);
        *(u32x2*)(sVt + (8 * dseg + d) * TA_VP + 4 * kq) = o;
      }
    }
    if (tid < TL_CT) sCnt[tid] = (float)kcounts[(size_t)h * TA_CK + tc * TL_CT + tid];
    __syncthreads();
    f32x16 S[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const uint16_t* cr = sC + (32 * kb + jl) * TL_CP + 8 * hh;
      S[kb] = zero16();
      S[kb] = Mfma<F16T>::run(*(const u32x4*)(cr), qb0, S[kb]);
      S[kb] = Mfma<F16T>::run(*(const u32x4*)(cr + 16), qb1, S[kb]);
    }
    float mx = -__builtin_inff();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int a = 0; a < 16; ++a) {
        S[kb][a] = h2f(f2h(S[kb][a]));  // scores are fp16, as in selection
        mx = fmaxf(mx, S[kb][a]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f((m - mnew) * L2E);
    m = mnew;
    const uint32_t uw0 = ur[2 * tc], uw1 = ur[2 * tc + 1];
    float ps = 0.f;
    u32x4 pb[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const uint32_t uw = kb ? uw1 : uw0;
#pragma unroll
      for (int a = 0; a < 16; a += 2) {
        const int b0 = 8 * (a / 4) + 4 * hh + (a % 4);
        const bool in0 = (uw >> b0) & 1u, in1 = (uw >> (b0 + 1)) & 1u;
        const float p0 = in0 ? 0.f : __builtin_amdgcn_exp2f((S[kb][a] - mnew) * L2E);
        const float p1 = in1 ? 0.f : __builtin_amdgcn_exp2f((S[kb][a + 1] - mnew) * L2E);
        ps = fmaf(p0, sCnt[32 * kb + b0], ps);
        ps = fmaf(p1, sCnt[32 * kb + b0 + 1], ps);
        pb[2 * kb + a / 8][(a % 8) / 2] = pack2(f2h(p0), f2h(p1));
      }
    }
    phi = phi * alpha + ps;
    if (alpha != 1.0f) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int a = 0; a < 16; ++a) O[nb][a] *= alpha;
    }
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const uint16_t* vr = sVt + (32 * nb + jl) * TA_VP + 4 * hh;
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        const u32x2 lo = *(const u32x2*)(vr + 16 * mm);
        const u32x2 hi = *(const u32x2*)(vr + 16 * mm + 8);
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        O[nb] = Mfma<F16T>::run(a, pb[mm], O[nb]);
      }
    }
  }
  if (!ok) return;
  phi += __shfl_xor(phi, 32, 64);
  const float tw = *tailw;
  const float lm = lam[h];
  const float le = attn_lse[(size_t)h * N + j] * 0.6931471805599453f;
  float ex, st;
  if (le >= m) {
    ex = 1.0f;
    st = __expf(m - le);
  } else {
    ex = __expf(le - m);
    st = 1.0f;
  }
  const float ph = st * phi;
  const bool bad = ph <= 1.0e-6f * ex;
  const float den = fmaxf(ex + ph * tw, 1.0e-12f);
  const float wx = ex / den, wt = st * tw * lm / den;
  const uint16_t* ar = attn_out + ((size_t)h * N + j) * TA_D;
  uint16_t* orow = out + ((size_t)h * N + orig) * TA_D;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * nb + 8 * g + 4 * hh;
      const u32x2 av = *(const u32x2*)(ar + d0);
      u32x2 ov = av;
      if (!bad) {
        float x[4];
        x[0] = T::to_f((uint16_t)(av[0] & 0xffff));
        x[1] = T::to_f((uint16_t)(av[0] >> 16));
        x[2] = T::to_f((uint16_t)(av[1] & 0xffff));
        x[3] = T::to_f((uint16_t)(av[1] >> 16));
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = fmaf(wt, O[nb][4 * g + e], wx * x[e]);
        ov[0] = pack2(T::from_f(x[0]), T::from_f(x[1]));
        ov[1] = pack2(T::from_f(x[2]), T::from_f(x[3]));
      }
      *(u32x2*)(orow + d0) = ov;
    }
}

// ---------------------------------------------------------------------------
// entry points
// ---------------------------------------------------------------------------
static int check_dtype(int dtype) { return dtype == T2T_F16 || dtype == T2T_BF16; }

extern "C" int t2t_tile_attn_exact(const void* q, const void* kp, const void* vp, int dtype,
                                   const int32_t* kcounts, const int32_t* unip,
                                   const int32_t* qperm, const int32_t* plan, void* attn_out,
                                   float* lse, int H, int N, int CQ, void* stream) {
  T2T_REQUIRE(q && kp && vp && kcounts && unip && qperm && plan && attn_out && lse,
              "tile_attn_exact: null pointer");
  T2T_REQUIRE(check_dtype(dtype), "tile_attn_exact: dtype %d", dtype);
  T2T_REQUIRE(H > 0 && N > 0 && CQ > 0, "tile_attn_exact: H=%d N=%d CQ=%d", H, N, CQ);
  PlanView p = plan_view((int32_t*)plan, H, N, CQ);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == T2T_F16)
    launch_attn<F16T, false>(q, kp, vp, unip, qperm, kcounts, p, attn_out, lse, nullptr, nullptr,
                             nullptr, nullptr, nullptr, nullptr, H, N, CQ, st);
  else
    launch_attn<BF16T, false>(q, kp, vp, unip, qperm, kcounts, p, attn_out, lse, nullptr, nullptr,
                              nullptr, nullptr, nullptr, nullptr, H, N, CQ, st);
  T2T_LAUNCH_CHECK("tile_attn_exact");
  return T2T_OK;
}

extern "C" int t2t_tail_merge(const void* attn_out, const float* lse, const void* QU,
                              const void* cks, const void* sumv, const int32_t* kcounts,
                              const int32_t* unip, const int32_t* qlab, const int32_t* qperm,
                              const float* lam, const float* tailw_dev, void* out, int dtype, int H,
                              int N, int CQ, void* stream) {
  T2T_REQUIRE(attn_out && lse && QU && cks && sumv && kcounts && unip && qlab && qperm && lam &&
                  tailw_dev && out,
              "tail_merge: null pointer");
  T2T_REQUIRE(check_dtype(dtype), "tail_merge: dtype %d", dtype);
  T2T_REQUIRE(H > 0 && N > 0 && CQ > 0, "tail_merge: H=%d N=%d CQ=%d", H, N, CQ);
  const dim3 grid(cdiv(N, 128), H);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == T2T_F16)
    hipLaunchKernelGGL(tail_kernel<F16T>, grid, dim3(256), 0, st, (const uint16_t*)attn_out, lse,
                       (const uint16_t*)QU, (const uint16_t*)cks, (const uint16_t*)sumv, kcounts,
                       (const uint32_t*)unip, qlab, qperm, lam, tailw_dev, (uint16_t*)out, N, CQ);
  else
    hipLaunchKernelGGL(tail_kernel<BF16T>, grid, dim3(256), 0, st, (const uint16_t*)attn_out, lse,
                       (const uint16_t*)QU, (const uint16_t*)cks, (const uint16_t*)sumv, kcounts,
                       (const uint32_t*)unip, qlab, qperm, lam, tailw_dev, (uint16_t*)out, N, CQ);
  T2T_LAUNCH_CHECK("tail_merge");
  return T2T_OK;
}

extern "C" size_t t2t_tile_attn_ws_bytes(int H, int N, int dtype) {
  (void)H;
  (void)N;
  (void)dtype;
  return 0;  // the fused kernel keeps the exact part in registers
}

extern "C" int t2t_tile_attn_run_planned(const void* q, const void* kp, const void* vp, int dtype,
                                         const int32_t* qcounts, const int32_t* kcounts,
                                         const int32_t* unip, const void* QU, const void* cks,
                                         const void* sumv, const float* lam, const int32_t* qlab,
                                         const int32_t* qperm, const float* tailw_dev, void* out,
                                         int32_t* plan, int rebuild_plan, int H, int N, int CQ,
                                         void* ws, size_t ws_bytes, void* stream) {
  (void)ws;
  (void)ws_bytes;
  T2T_REQUIRE(q && kp && vp && qcounts && kcounts && unip && QU && cks && sumv && lam && qlab &&
                  qperm && tailw_dev && out && plan,
              "tile_attn_run_planned: null pointer");
  T2T_REQUIRE(check_dtype(dtype), "tile_attn_run_planned: dtype %d", dtype);
  T2T_REQUIRE(H > 0 && N > 0 && CQ > 0, "tile_attn_run_planned: H=%d N=%d CQ=%d", H, N, CQ);
  hipStream_t st = (hipStream_t)stream;
  if (rebuild_plan) {
    const int rc = t2t_tile_plan(qcounts, kcounts, unip, plan, H, N, CQ, stream);
    if (rc) return rc;
  }
  PlanView p = plan_view(plan, H, N, CQ);
  if (dtype == T2T_F16)
    launch_attn<F16T, true>(q, kp, vp, unip, qperm, kcounts, p, nullptr, nullptr, QU, cks, sumv,
                            lam, tailw_dev, out, H, N, CQ, st);
  else
    launch_attn<BF16T, true>(q, kp, vp, unip, qperm, kcounts, p, nullptr, nullptr, QU, cks, sumv,
                             lam, tailw_dev, out, H, N, CQ, st);
  T2T_LAUNCH_CHECK("tile_attn_run_planned");
  return T2T_OK;
}
