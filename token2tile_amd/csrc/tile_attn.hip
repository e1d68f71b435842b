// S5/S6: task planning, exact attention over each query cluster's union of
// key clusters, and the centroid residual + merge (gfx950, MFMA 32x32x16).
//
// Exact attention (one work-group per task of <= 128 sorted queries of one
// query cluster, 4 waves x 32 queries, two work-groups per CU):
//   * the union is turned into runs of cluster-ordered key rows in LDS, and
//     the vp rows of every 64-key tile are derived from them in parallel (K
//     rows through kperm, or from the cluster-ordered kp);
//   * K and V tiles are gathered by LDS DMA into a double-buffered ring, row
//     major with an XOR swizzle; tile t is consumed while tile t+1 is in
//     flight.  In tasks of four query waves every wave stages a quarter of
//     each tile, one barrier per tile; in smaller tasks the last wave (which
//     holds no queries) stages every tile and publishes it through an LDS
//     flag, and the query waves report each buffer they finish through an LDS
//     counter, so no wave waits for the slowest one at every tile;
//   * S^T = K Q^T and O^T = V^T P^T on MFMA, so every lane owns one query: the
//     online-softmax max/sum need one cross-half exchange, and the per-query
//     rescale of O touches only the lane's own registers; the score chains
//     read K four steps ahead, and V^T operands come from transposing LDS
//     reads issued in inline assembly one dim block ahead;
//   * the running max advances with a margin, so O is rescaled only when a
//     tile raises the max by more than the margin.
// Residual + merge (a separate kernel, one work-group per 128 consecutive
// sorted queries): the same structure over the 2048 centroids (K = cks,
// V = sumv, staged from a per-call tile image), each lane masking its own
// query cluster's union, then the merge with the exact part.
#include "t2t_common.h"
#include <type_traits>

#define TA_D 128
#define TA_CK 2048
#define TA_QT 128   // queries per task (4 waves x 32)
#define TA_WAVES 4
#define TA_KT 64    // keys per tile

// ---------------------------------------------------------------------------
// plan layout (int32): k_off [H][2049] | kvlen [H][CQ] | ntask [H] |
//                      tasks [H][maxT][4] = (cluster, sorted start, rows, cluster task rows)
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
  // task list: cluster t splits into ceil(n / QT) tasks of whole waves
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
      // the cluster's ceil(n / 32) waves of 32 queries are dealt evenly over
      // its tasks; only the last task holds a partial wave, so the tasks pad
      // no more query rows than the cluster needs (an even split of the rows
      // would pad every task's last wave)
      const int nw = (n + 31) / 32;
      const int base = nw / nt, rem = nw % nt;
      int s = qex;
      for (int i = 0; i < nt; ++i) {
        const int rows = min(32 * (base + (i < rem ? 1 : 0)), qex + n - s);
        int32_t* tk = th + (size_t)(tex + i) * 4;
        tk[0] = t;
        tk[1] = s;
        tk[2] = rows;
        tk[3] = 32 * (base + (rem > 0 ? 1 : 0));  // the cluster's largest task
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
  // LPT order: descending (largest task rows of the cluster) x kv_len, ties
  // by lower task index, so the tasks of one query cluster, which stream the
  // same key/value union, stay next to each other and run on one XCD
  int P2 = 2;
  while (P2 < nT) P2 <<= 1;
  for (int i = tid; i < P2; i += 1024) {
    unsigned long long key = 0ull;
    if (i < nT) {
      const int32_t* tk = th + (size_t)i * 4;
      unsigned long long work =
          (unsigned long long)tk[3] * (unsigned long long)kvlen[(size_t)h * CQ + tk[0]];
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

// map a linear block id to a task: blocks are dealt to the 8 XCDs round
// robin, so groups of 8 consecutive tasks (the tasks of one query cluster sit
// next to each other in the task list) run on one XCD and share its L2, while
// all XCDs sweep the task list together and keep to the same head's K/V in the
// shared last-level cache.  The grid is a multiple of 64 blocks.
__device__ inline int xcd_remap(int bid, int total) {
  (void)total;
  const int r = bid / 8;
  return (r / 8) * 64 + (bid % 8) * 8 + r % 8;
}

#define T2T_SPIN_CAP (1 << 20)  // polls before a producer/consumer wait gives up
#define TA_MARGIN 3.0f   // log2 units of headroom when the exact-part max advances
// a tile is redone with a new max when one lane's weight sum passes this: far
// inside the range of bf16 P (fp32 exponents), below fp16's largest value
#define TA_WLIM (T::code == T2T_BF16 ? 0x1p64f : 0x1p14f)
#define TL_MARGIN 2.0f   // natural-log units of headroom for the residual max
#define TL_CT 64         // centroids per residual tile
#define TL_CP 40         // residual centroid tile pitch (halves)

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// LDS tile layouts (no padding, XOR swizzles keep the MFMA operand reads
// conflict free):
//   sK  [64 keys][128 dims]: 16-byte chunk c of row r lives at chunk c ^ (r & 15)
//   sV  [64 keys][128 dims]: chunk c of row r at chunk c ^ sv_swz(r)
//   sVt [128 dims][64 keys]: the 4-key granules a lane feeds to one MFMA
//     (g = 4 m + h and 4 m + 2 + h) are stored side by side, so the operand is
//     one 16-byte read: granule g sits in 16-byte unit (g & ~3) / 2 + (g & 1),
//     half (g >> 1) & 1.  Rows are padded to 144 bytes: 16 lanes reading one
//     unit of 16 consecutive dims start on banks 36 d mod 64, all distinct,
//     and every operand of a lane is one base address plus a constant.
__device__ inline int sk_off(int row, int chunk) { return row * 128 + 8 * (chunk ^ (row & 15)); }
// sV [64 keys][128 dims], row-major, read only by the transposing reads: 16-byte
// chunk c of key r lives at chunk c ^ sv_swz(r).  One such read has the 32 lanes
// of a half-wave address 4 consecutive keys (r % 4 = 0..3) x chunk bits 0-1
// (8-byte half by lane parity); moving r % 4 into chunk bits 2-3 puts the half-wave
// on all 64 banks exactly once.  (The K swizzle, r & 15, would overlap r % 4 with
// chunk bits 0-1 and leave the half-wave on 16 banks: 4-way conflicts.)
__device__ inline int sv_swz(int row) { return (row & 3) << 2; }
#define VT_PITCH 72  // halves per sVt row: 64 keys + one unit of padding
__device__ inline int vt_unit_off(int dim, int unit) { return dim * VT_PITCH + 8 * unit; }
__device__ inline int vt_gran_off(int dim, int g) {
  return vt_unit_off(dim, ((g & ~3) >> 1) + (g & 1)) + 4 * ((g >> 1) & 1);
}

__device__ inline float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
// bitfield insert: (m & a) | (~m & b), one v_bfi_b32.  Only ever applied to
// values produced by ordinary VALU instructions (never straight to an MFMA
// result: the compiler's wait states for reading MFMA results do not cover
// inline assembly).
__device__ inline uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(a), "v"(b));
  return r;
}
// (b.lo16 << 16) | a.lo16 and (b.hi16 << 16) | a.hi16
__device__ inline uint32_t pack_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ inline uint32_t pack_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }
// keeps the compiler from if-converting a rarely taken block into selects
#define T2T_REAL_BRANCH() asm volatile("" ::: "memory")

// One work-group (4 waves, 32 queries each) per task of <= 128 queries, two
// work-groups per CU.  MODE 0: attn_out and lse (log2 units) in sorted order.
// MODE 1: the exact output at the original rows of out, lse in sorted order
// MODE 2: as MODE 1, with the K gather fused: kp is k in its original order and
// key position p of cluster order reads row kperm[p] (no separate kp = k[kperm])
// MODE 3: as MODE 2, with the V gather fused as well: vp is v in its original
// order, read through kperm like K (no V_sorted)
// (the residual kernel merges into out in place).
template <typename T, int MODE>
__global__ __launch_bounds__(TA_WAVES * 64, 2) void attn_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kp,
    const uint16_t* __restrict__ vp, const uint32_t* __restrict__ unip,
    const int32_t* __restrict__ qperm, const int32_t* __restrict__ kcounts,
    const int32_t* __restrict__ k_off, const int32_t* __restrict__ ntask,
    const int32_t* __restrict__ tasks, uint16_t* __restrict__ attn_out, float* __restrict__ lse,
    uint16_t* __restrict__ out, const int32_t* __restrict__ kperm, int H, int N, int CQ, int maxT,
    long long sqh, long long sqn, long long skh, long long skn, long long soh, long long son,
    long long svh, long long svn) {
  // row n of head h of q / k (MODE 2) / out (MODE 1, 2) sits at base + h s_h + n s_n
  // (elements): [H, N, 128] contiguous or a strided view such as token-major [N, H, 128]
  constexpr bool KG = MODE >= 2;
  constexpr bool VG = MODE == 3;
  // two separate arrays (not one [2][...] array): the K DMA into one buffer
  // must not be taken as a possible writer of the other one, or every read of
  // the tile in use would wait for the loads of the tile in flight
  __shared__ __attribute__((aligned(1024))) uint16_t sK0[TA_KT * 128];
  __shared__ __attribute__((aligned(1024))) uint16_t sK1[TA_KT * 128];
  __shared__ __attribute__((aligned(1024))) uint16_t sV0[TA_KT * 128];
  __shared__ __attribute__((aligned(1024))) uint16_t sV1[TA_KT * 128];
  // runs of the union: first key position (cum) and first kp/vp row of each
  // run, as 24-bit values (16-bit low part + 8-bit high part; N < 2^24), so
  // the index builder reads only LDS
  __shared__ uint16_t runCumLo[TA_CK + 1], runRowLo[TA_CK];
  __shared__ uint8_t runCumHi[TA_CK + 1], runRowHi[TA_CK];
  // byte offsets of each tile position's K and V source rows from the head
  // base (built once per tile by the index wave, so the DMA issue is one add
  // per row): sIdx for the cluster-ordered kp / vp rows (256 bytes each),
  // sIdxK / sIdxV for rows read in place through kperm (MODE >= 2 / 3)
  __shared__ uint32_t sIdx[2][TA_KT];
  __shared__ uint32_t sIdxK[KG ? 2 : 1][KG ? TA_KT : 1];
  __shared__ uint32_t sIdxV[VG ? 2 : 1][VG ? TA_KT : 1];
  __shared__ int bMark[TA_KT];
  // producer/consumer form (tasks whose last wave holds no queries): the tile
  // last published in each buffer (tile + 1) and the count of consumer waves
  // done with each buffer, both monotonic
  // sAbort: set when a wait passes T2T_SPIN_CAP polls; every later wait of the
  // work-group then returns at once, so a broken handshake ends the kernel
  // (with NaN in the task's output) instead of hanging it
  __shared__ int sReady[2], sDone[2], sAbort;
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
      const int row0 = ko[8 * tid + j];
      runCumLo[r] = (uint16_t)p;
      runCumHi[r] = (uint8_t)(p >> 16);
      runRowLo[r] = (uint16_t)row0;
      runRowHi[r] = (uint8_t)(row0 >> 16);
      ++r;
      p += cnts[j];
    }
  }
  if (tid == 0) {
    runCumLo[nrun] = (uint16_t)kvlen;
    runCumHi[nrun] = (uint8_t)(kvlen >> 16);
  }
  auto run_cum = [&](int r) { return (int)runCumLo[r] | ((int)runCumHi[r] << 16); };
  auto run_row = [&](int r) { return (int)runRowLo[r] | ((int)runRowHi[r] << 16); };

  const int qrow = wave * 32 + jl;  // query row inside the task
  const bool qok = qrow < qrows;
  const bool wave_active = wave * 32 < qrows;
  const size_t obase = (size_t)h * N + qs;  // sorted-order rows of the task
  const int orig = qperm[obase + (qok ? qrow : 0)];
  // ---- O^T += V^T P^T over one 64-key tile, V^T read from the row-major V
  // tile by two transposing reads per operand.  In a 16-lane group, lane i of
  // ds_read_b64_tr_b16 gets, in slot k, element i % 4 of the 8 bytes that lane
  // 4 k + i / 4 addresses.  Lane l addresses key 16 mm + 8 r + 4 hh +
  // (l % 16) / 4 at dims D + 4 (l % 4) .. + 3, D = 32 nb + 16 ((l / 16) % 2),
  // and so receives dim D + l % 16 of keys 16 mm + 8 r + 4 hh + 0 .. 3: the
  // operand elements t = 4 r + k, which hold keys 8 (t / 4) + 4 hh + t % 4 of
  // the k-step, the order the P fragments are packed in.  The swizzle of key
  // 16 mm + 8 r + trkey depends on trkey alone, so one address per dim block
  // nb serves all eight reads of the block, with mm and r as immediate
  // offsets of (16 mm + 8 r) * 256 bytes.
  const int trkey = 4 * hh + ((lane & 15) >> 2);
  const int trdim = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  // P.V with the transposing reads in inline assembly: the compiler's own
  // form of this read waits on every in-flight vector-memory load (the next
  // tile's K/V DMA) before it, cutting that DMA's latency budget to half a
  // tile.  The reads of dim block nb + 1 are issued before the MFMAs of nb,
  // and an explicit lgkmcnt wait that names nb's fragments as its operands
  // orders those MFMAs after their data (no other LDS access is in flight).
  auto pv = [&](f32x16 (&Oa)[4], const uint16_t* sVb, const u32x4 (&pb)[4]) __attribute__((always_inline)) {
    const uint32_t vbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint16_t*)sVb;
    uint32_t ad[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
      ad[nb] = vbase + 2u * (uint32_t)(trkey * 128 + 8 * ((4 * nb + (trdim >> 3)) ^ sv_swz(trkey)) + (trdim & 7));
    u32x2 fr[2][8];
    auto rd8 = [&](u32x2 (&f)[8], uint32_t a) __attribute__((always_inline)) {
      asm volatile(
          "ds_read_b64_tr_b16 %0, %8\n\t"
          "ds_read_b64_tr_b16 %1, %8 offset:2048\n\t"
          "ds_read_b64_tr_b16 %2, %8 offset:4096\n\t"
          "ds_read_b64_tr_b16 %3, %8 offset:6144\n\t"
          "ds_read_b64_tr_b16 %4, %8 offset:8192\n\t"
          "ds_read_b64_tr_b16 %5, %8 offset:10240\n\t"
          "ds_read_b64_tr_b16 %6, %8 offset:12288\n\t"
          "ds_read_b64_tr_b16 %7, %8 offset:14336"
          : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]),
            "=&v"(f[6]), "=&v"(f[7])
          : "v"(a));
    };
    __builtin_amdgcn_sched_barrier(0);
    rd8(fr[0], ad[0]);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      u32x2 (&f)[8] = fr[nb & 1];
      if (nb + 1 < 4) {
        rd8(fr[(nb + 1) & 1], ad[nb + 1]);
        asm volatile("s_waitcnt lgkmcnt(8)"
                     : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]),
                       "+v"(f[6]), "+v"(f[7]));
      } else {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]),
                       "+v"(f[6]), "+v"(f[7]));
      }
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        const u32x4 a = {f[2 * mm][0], f[2 * mm][1], f[2 * mm + 1][0], f[2 * mm + 1][1]};
        Oa[nb] = Mfma<T>::run(a, pb[mm], Oa[nb]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto rescale = [&](f32x16 (&Oa)[4], float alpha) __attribute__((always_inline)) {
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
      const uint16_t* qr = q + (size_t)h * sqh + (size_t)orig * sqn + 8 * hh;
#pragma unroll
      for (int s = 0; s < 8; ++s) qb[s] = *(const u32x4*)(qr + 16 * s);
    }
    const char* kh = (const char*)(kp + (KG ? (size_t)h * skh : (size_t)h * N * TA_D));
    // byte offsets of K rows from the head base stay 32-bit (the entry point
    // checks (N - 1) * row stride fits): 64-bit address math here cost 3.6%
    const uint32_t krow_bytes = KG ? (uint32_t)(skn * 2) : 256u;
    const char* vh = (const char*)(vp + (VG ? (size_t)h * svh : (size_t)h * N * TA_D));
    const uint32_t vrow_bytes = VG ? (uint32_t)(svn * 2) : 256u;
    const int ntile = (kvlen + TA_KT - 1) / TA_KT;
    // source rows of tile `tile` -> sIdx[tile & 1]; past the end -> row 0
    // (its keys are masked and its values multiply a zero probability).
    // Built by the last wave (idle in tasks of <= 96 rows) without loops:
    // every run is non-empty, so runs r0 .. r0 + 63 cover the tile, r0 being
    // the run that holds its first position.  Lane j reads run r0 + j and
    // marks the tile slot where that run starts; a prefix max over the marks
    // gives each position its run.
    int r0 = 0;
    // MODE >= 2: the K rows of the tile last built, loaded from kperm by the
    // index wave and stored (as byte offsets) to sIdxK / sIdxV after the next
    // wait on the memory counter
    int kpend = 0;
    const int32_t* kph = KG ? kperm + (size_t)h * N : nullptr;
    auto build_idx = [&](int tile) __attribute__((always_inline)) {
      if (wave == TA_WAVES - 1) {
        const int base = tile * TA_KT;
        const int r = r0 + lane;
        int cs = 0x7fffffff, rw = 0;
        if (r < nrun) {
          cs = run_cum(r);
          rw = run_row(r);
        }
        const int st = cs - base;  // lane 0: <= 0; other valid lanes: > 0
        bMark[lane] = 0;
        __builtin_amdgcn_wave_barrier();
        if (lane == 0 || st < TA_KT) bMark[lane == 0 ? 0 : st] = lane + 1;
        __builtin_amdgcn_wave_barrier();
        const int k = wave_incl_max(bMark[lane] - 1);
        const int pos = base + lane;
        const int ck = __shfl(cs, k, 64), rk = __shfl(rw, k, 64);
        const int vrow = pos < kvlen ? rk + pos - ck : 0;
        sIdx[tile & 1][lane] = (uint32_t)vrow << 8;
        if constexpr (KG) kpend = pos < kvlen ? kph[vrow] : 0;
        // run holding the next tile's first position: the last run starting at
        // or before it.  The lanes see runs r0 .. r0 + 63 only; when all of
        // them qualify (64 runs of one key each), run r0 + 64 may start exactly
        // there too and is checked separately.
        const int seen = __popcll(__ballot(st <= TA_KT));
        int nxt = r0 + seen - 1;
        if (seen == 64 && r0 + 64 < nrun && run_cum(r0 + 64) <= base + TA_KT) nxt = r0 + 64;
        r0 = nxt;
      }
    };
    auto flush_k = [&](int tile) __attribute__((always_inline)) {
      if constexpr (KG)
        if (wave == TA_WAVES - 1) {
          sIdxK[tile & 1][lane] = (uint32_t)kpend * krow_bytes;
          if constexpr (VG) sIdxV[tile & 1][lane] = (uint32_t)kpend * vrow_bytes;
        }
    };
    // K and V tiles via LDS DMA (each wave instruction fills 4 whole rows, the
    // lane fetching the 16-byte chunk that belongs at its swizzled position)
    auto issue = [&](int tile, auto BUF) __attribute__((always_inline)) {
      constexpr int buf = decltype(BUF)::value;
      uint16_t* sKb = buf ? sK1 : sK0;
      uint16_t* sVb = buf ? sV1 : sV0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int blk = 4 * i + wave;
        const int row = 4 * blk + (lane >> 4);
        const uint32_t base = sIdx[buf][row];
        const uint32_t kbase = KG ? sIdxK[buf][row] : base;
        const uint32_t offk = kbase + 16u * ((lane & 15) ^ (row & 15));
        const uint32_t vbase = VG ? sIdxV[buf][row] : base;
        const uint32_t offv = vbase + 16u * ((lane & 15) ^ sv_swz(row));
        __builtin_amdgcn_global_load_lds((const glb_void_t*)(kh + offk),
                                         (lds_void_t*)(sKb + blk * 4 * 128), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const glb_void_t*)(vh + offv),
                                         (lds_void_t*)(sVb + blk * 4 * 128), 16, 0, 0);
      }
    };
    // one 64-key tile of the online softmax; MASK: the last, partial tile
    auto tile_step = [&](auto BUF, int valid, auto MASK) __attribute__((always_inline)) {
      constexpr int buf = decltype(BUF)::value;
      const uint16_t* sKb = buf ? sK1 : sK0;
      // scores of the two 32-key halves as two interleaved MFMA chains, each
      // chain's K fragment read four steps ahead.  The scheduling barriers
      // keep that order: left alone, the compiler read one chain ahead into
      // spare registers and fed the other through a single buffer, each MFMA
      // of it waiting on its own LDS read.
      f32x16 S[2] = {zero16(), zero16()};
      auto rdk = [&](int kb, int s) __attribute__((always_inline)) {
        return *(const u32x4*)(sKb + sk_off(32 * kb + jl, 2 * s + hh));
      };
      constexpr int KD = 4;  // read-ahead depth in k-steps
      u32x4 f0[KD], f1[KD];
#pragma unroll
      for (int s = 0; s < KD; ++s) {
        f0[s] = rdk(0, s);
        f1[s] = rdk(1, s);
      }
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        __builtin_amdgcn_sched_barrier(0);
        S[0] = Mfma<T>::run(f0[s % KD], qb[s], S[0]);
        S[1] = Mfma<T>::run(f1[s % KD], qb[s], S[1]);
        if (s + KD < 8) {
          f0[s % KD] = rdk(0, s + KD);
          f1[s % KD] = rdk(1, s + KD);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (decltype(MASK)::value) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int a = 0; a < 16; ++a)
            if (32 * kb + 8 * (a / 4) + 4 * hh + (a % 4) >= valid) S[kb][a] = -__builtin_inff();
      }
      // weights against the current m, without a per-tile max: exp2 scales
      // exactly, so m only has to keep the weights in the range of T.  A tile
      // whose weights leave it (the first one, m = -inf, or scores far above
      // every earlier tile) is redone with m moved past its max, the sums so
      // far rescaled (the reference's lazy max, taken only when needed)
      u32x4 pb[4];
      auto expo = [&](float nm) __attribute__((always_inline)) {
        float acc = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int a = 0; a < 16; a += 2) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(S[kb][a], c, nm));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(S[kb][a + 1], c, nm));
            const uint32_t pk = Pk<T>::pack(p0, p1);
            acc = Pk<T>::sum2(pk, acc);
            pb[2 * kb + a / 8][(a % 8) / 2] = pk;
          }
        return acc;
      };
      float lt = expo(-m);
      if (__builtin_amdgcn_readfirstlane((int)(__ballot(!(lt <= TA_WLIM)) != 0ull))) {
        T2T_REAL_BRANCH();
        float mr = -__builtin_inff();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int a = 0; a < 16; a += 2) mr = vmax(mr, vmax(S[kb][a], S[kb][a + 1]));
        mr = half_max(mr);
        const float mx = mr * c;
        const float mnew = mx > m ? mx + TA_MARGIN : m;
        const float alpha = __builtin_amdgcn_exp2f(m - mnew);
        m = mnew;
        lsum *= alpha;
        rescale(O, alpha);
        lt = expo(-m);
      }
      lsum += lt;
      pv(O, buf ? sV1 : sV0, pb);
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    if (tid < 2) {
      sReady[tid] = 0;
      sDone[tid] = 0;
    }
    if (tid == 0) sAbort = 0;
    __syncthreads();  // runs visible
    if (qrows <= 32 * (TA_WAVES - 1)) {
      // the last wave stages every tile (all 16 row groups of K and V) and
      // publishes it; the consumer waves wait only for the tile they read and
      // report when they are done with a buffer
      const int nact = (qrows + 31) >> 5;
      auto issue_all = [&](int tile, auto BUF) __attribute__((always_inline)) {
        constexpr int buf = decltype(BUF)::value;
        uint16_t* sKb = buf ? sK1 : sK0;
        uint16_t* sVb = buf ? sV1 : sV0;
#pragma unroll
        for (int blk = 0; blk < 16; ++blk) {
          const int row = 4 * blk + (lane >> 4);
          const uint32_t base = sIdx[buf][row];
          const uint32_t kbase = KG ? sIdxK[buf][row] : base;
          const uint32_t offk = kbase + 16u * ((lane & 15) ^ (row & 15));
          const uint32_t vbase = VG ? sIdxV[buf][row] : base;
          const uint32_t offv = vbase + 16u * ((lane & 15) ^ sv_swz(row));
          __builtin_amdgcn_global_load_lds((const glb_void_t*)(kh + offk),
                                           (lds_void_t*)(sKb + blk * 4 * 128), 16, 0, 0);
          __builtin_amdgcn_global_load_lds((const glb_void_t*)(vh + offv),
                                           (lds_void_t*)(sVb + blk * 4 * 128), 16, 0, 0);
        }
      };
      // poll an LDS word until ok(value); bounded (see sAbort)
      auto spin = [&](int* w, auto ok) __attribute__((always_inline)) {
        for (int n = 0;; ++n) {
          if (ok(__hip_atomic_load(w, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP))) return;
          if (n > T2T_SPIN_CAP ||
              __hip_atomic_load(&sAbort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) {
            if (lane == 0)
              __hip_atomic_store(&sAbort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            return;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      };
      auto publish = [&](int tile) __attribute__((always_inline)) {
        if (lane == 0)
          __hip_atomic_store(&sReady[tile & 1], tile + 1, __ATOMIC_RELEASE,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
      };
      if (wave == TA_WAVES - 1) {
        build_idx(0);
        flush_k(0);
        issue_all(0, B0{});
        if (ntile > 1) {
          build_idx(1);
          flush_k(1);
          issue_all(1, B1{});
        }
        if (ntile > 2) build_idx(2);
        __builtin_amdgcn_s_waitcnt(0);
        publish(0);
        for (int t = 0; t + 1 < ntile; ++t) {
          __builtin_amdgcn_s_waitcnt(0);  // tile t + 1 (and the kperm rows of t + 2) landed
          publish(t + 1);
          if (t + 2 < ntile) {
            flush_k(t + 2);
            const int want = nact * ((t >> 1) + 1);
            spin(&sDone[t & 1], [&](int v) { return v >= want; });
            if (t & 1)
              issue_all(t + 2, B1{});
            else
              issue_all(t + 2, B0{});
            if (t + 3 < ntile) build_idx(t + 3);
          }
        }
      } else if (wave < nact) {
        auto consume = [&](int tile, auto BUF, int valid, auto MASK) __attribute__((always_inline)) {
          constexpr int buf = decltype(BUF)::value;
          spin(&sReady[buf], [&](int v) { return v == tile + 1; });
          tile_step(BUF, valid, MASK);
          if (lane == 0)
            __hip_atomic_fetch_add(&sDone[buf], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        };
        const int nfull = (kvlen % TA_KT) ? ntile - 1 : ntile;
        int tile = 0;
        for (; tile + 2 <= nfull; tile += 2) {
          consume(tile, B0{}, TA_KT, std::false_type{});
          consume(tile + 1, B1{}, TA_KT, std::false_type{});
        }
        if (tile < nfull) consume(tile++, B0{}, TA_KT, std::false_type{});
        if (tile < ntile) {
          const int valid = kvlen - tile * TA_KT;
          if (tile & 1)
            consume(tile, B1{}, valid, std::true_type{});
          else
            consume(tile, B0{}, valid, std::true_type{});
        }
        // a wait that gave up leaves the output NaN, not silently wrong
        if (__hip_atomic_load(&sAbort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP))
          lsum = __builtin_nanf("");
      }
    } else {
    // tasks of four waves: every wave stages a quarter of each tile, one
    // barrier per tile
    build_idx(0);
    flush_k(0);
    if (ntile > 1) {
      build_idx(1);
      flush_k(1);
    }
    __syncthreads();
    issue(0, B0{});
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (ntile > 1) issue(1, B1{});
    if (ntile > 2) build_idx(2);
    // one full tile held in buffer BUF: consume it, stage the V of the next
    // tile, wait for the next tile's K, then start the tile after it
    auto body = [&](int tile, auto BUF) __attribute__((always_inline)) {
      constexpr int buf = decltype(BUF)::value;
      if (wave_active) tile_step(BUF, TA_KT, std::false_type{});
      __builtin_amdgcn_s_waitcnt(0);  // K and V DMA of tile + 1 landed (and kperm of tile + 2)
      if (tile + 2 < ntile) flush_k(tile + 2);
      __syncthreads();
      if (tile + 2 < ntile) issue(tile + 2, BUF);
      if (tile + 3 < ntile) build_idx(tile + 3);
    };
    // full tiles two at a time, so that each buffer is a compile-time
    // constant; a partial last tile is peeled after the loop (a masked copy of
    // the tile body inside the loop would raise its register pressure)
    const int nfull = (kvlen % TA_KT) ? ntile - 1 : ntile;
    int tile = 0;
    for (; tile + 2 <= nfull; tile += 2) {
      body(tile, B0{});
      body(tile + 1, B1{});
    }
    if (tile < nfull) body(tile++, B0{});
    if (tile < ntile && wave_active) {
      const int valid = kvlen - tile * TA_KT;
      if (tile & 1)
        tile_step(B1{}, valid, std::true_type{});
      else
        tile_step(B0{}, valid, std::true_type{});
    }
    }
  }
  const float lt = half_sum(lsum);
  const float inv = kvlen > 0 ? 1.0f / lt : 0.f;
  const float lse2 = kvlen > 0 ? m + __log2f(lt) : -__builtin_inff();
  // exact output of the lane's 64 dims, rounded to T as the exact buffer
  // holds it: sorted-order attn_out (exact-only kernel) or, for the fused
  // kernel, the original row of out, read back by the merge
  if (qok) {
    uint16_t* orow =
        MODE != 0 ? out + (size_t)h * soh + (size_t)orig * son : attn_out + (obase + qrow) * TA_D;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(u32x2*)(orow + 32 * nb + 8 * g + 4 * hh) =
            u32x2{Pk<T>::pack(O[nb][4 * g] * inv, O[nb][4 * g + 1] * inv),
                  Pk<T>::pack(O[nb][4 * g + 2] * inv, O[nb][4 * g + 3] * inv)};
  }
  if (qok && hh == 0) lse[obase + qrow] = lse2;
}

template <typename T, int MODE>
static void launch_attn(const void* q, const void* kp, const void* vp, const int32_t* unip,
                        const int32_t* qperm, const int32_t* kcounts, const PlanView& p,
                        void* attn_out, float* lse, void* out, int H, int N, int CQ,
                        hipStream_t st, const int32_t* kperm = nullptr, long long sqh = -1,
                        long long sqn = TA_D, long long skh = -1, long long skn = TA_D,
                        long long soh = -1, long long son = TA_D, long long svh = -1,
                        long long svn = TA_D) {
  // default strides: [H, N, 128] contiguous
  if (sqh < 0) sqh = (long long)N * TA_D;
  if (svh < 0) svh = (long long)N * TA_D;
  if (skh < 0) skh = (long long)N * TA_D;
  if (soh < 0) soh = (long long)N * TA_D;
  const int total = H * p.maxT;
  const int grid = ((total + 63) / 64) * 64;
  hipLaunchKernelGGL((attn_kernel<T, MODE>), dim3(grid), dim3(TA_WAVES * 64), 0, st,
                     (const uint16_t*)q, (const uint16_t*)kp, (const uint16_t*)vp,
                     (const uint32_t*)unip, qperm, kcounts, p.k_off, p.ntask, p.tasks,
                     (uint16_t*)attn_out, lse, (uint16_t*)out, kperm, H, N, CQ, p.maxT, sqh, sqn,
                     skh, skn, soh, son, svh, svn);
}

// ---------------------------------------------------------------------------
// residual over the centroids outside each query's union + merge
// ---------------------------------------------------------------------------
// Centroid tile image, built once per call and staged by LDS DMA: per head,
// 32 tiles of 64 centroids, RT_BYTES each:
//   [0, 4096)      cks rows, 64 x 32 halves; 16-byte chunk c of row r sits at
//                  chunk c ^ ((r >> 2) & 3), so the MFMA operand reads of 16
//                  consecutive rows hit distinct banks
//   [4096, 22528)  sumv transposed, 128 dims x 64 centroids in the sVt layout
//                  (the padding unit of each row is never written or read)
#define RT_TILES (TA_CK / TL_CT)
#define RT_BYTES (4096 + 128 * VT_PITCH * 2)
#define RT_HALVES (RT_BYTES / 2)
static_assert(RT_BYTES % 1024 == 0, "the staging moves 1 KB per wave and instruction");
__device__ inline int rc_off(int r, int c) { return r * 32 + 8 * (c ^ ((r >> 2) & 3)); }

__global__ __launch_bounds__(256) void centroid_tiles_kernel(const uint16_t* __restrict__ cks,
                                                             const uint16_t* __restrict__ sumv,
                                                             uint16_t* __restrict__ tiles) {
  const int tc = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  uint16_t* dst = tiles + ((size_t)h * RT_TILES + tc) * RT_HALVES;
  const uint16_t* ch = cks + ((size_t)h * TA_CK + tc * TL_CT) * 32;
  const uint16_t* vh = sumv + ((size_t)h * TA_CK + tc * TL_CT) * TA_D;
  {
    const int r = tid >> 2, c = tid & 3;
    *(u32x4*)(dst + rc_off(r, c)) = *(const u32x4*)(ch + r * 32 + 8 * c);
  }
  // thread: 4 centroids (kq) x 8 dims (dseg), transposed into 4-centroid granules
  const int kq = tid >> 4, dseg = tid & 15;
  u32x4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = *(const u32x4*)(vh + (size_t)(4 * kq + i) * TA_D + 8 * dseg);
  uint16_t* vt = dst + 2048;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const u32x2 lo = {pack_lo(v[0][w], v[1][w]), pack_lo(v[2][w], v[3][w])};
    const u32x2 hi = {pack_hi(v[0][w], v[1][w]), pack_hi(v[2][w], v[3][w])};
    *(u32x2*)(vt + vt_gran_off(8 * dseg + 2 * w, kq)) = lo;
    *(u32x2*)(vt + vt_gran_off(8 * dseg + 2 * w + 1, kq)) = hi;
  }
}

// One work-group per 128 consecutive sorted queries (4 waves x 32, queries of
// several query clusters side by side): every lane masks the centroids of
// its own cluster's union, so all waves carry real rows.  The exact part is
// read from attn_out (sorted order, SRC_SORTED) or from the original rows of
// out, and the merged result is written to the original rows of out.
template <typename T, bool SRC_SORTED>
__global__ __launch_bounds__(256, 3) void resid_kernel(
    const uint16_t* __restrict__ exact, const float* __restrict__ lse2v,
    const uint16_t* __restrict__ QU, const uint16_t* __restrict__ tiles,
    const int32_t* __restrict__ kcounts, const uint32_t* __restrict__ unip,
    const int32_t* __restrict__ qlab, const int32_t* __restrict__ qperm,
    const float* __restrict__ lam, const float* __restrict__ tailw, uint16_t* __restrict__ out,
    int N, int CQ, long long soh, long long son) {
  __shared__ __attribute__((aligned(1024))) uint16_t sT0[RT_HALVES];
  __shared__ __attribute__((aligned(1024))) uint16_t sT1[RT_HALVES];
  // counts as fp16, ordered so that the 16 a lane weights in one 32-centroid
  // half are contiguous: centroid 64 t + 32 kb + 8 j + 4 hh + e sits at
  // 64 t + 32 kb + 16 hh + 4 j + e
  __shared__ __attribute__((aligned(16))) uint16_t sCnt[TA_CK];
  // row n of sMask: -inf where bit e of n is set, else 0 (the union mask of
  // four consecutive centroids)
  __shared__ __attribute__((aligned(16))) float sMask[16 * 4];
  const int h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int jl = lane & 31, hh = lane >> 5;
  const int row = blockIdx.x * 128 + wave * 32 + jl;  // sorted position
  const bool ok = row < N;
  const int orig = qperm[(size_t)h * N + (ok ? row : 0)];
  const uint32_t* ur = unip + ((size_t)h * CQ + qlab[(size_t)h * N + orig]) * (TA_CK / 32);
  u32x4 qu0, qu1;
  {
    const uint16_t* qr = QU + ((size_t)h * N + orig) * 32 + 8 * hh;
    qu0 = *(const u32x4*)(qr);
    qu1 = *(const u32x4*)(qr + 16);
  }
  const char* th = (const char*)(tiles + (size_t)h * RT_TILES * RT_HALVES) + wave * 1024 + lane * 16;
  auto issue = [&](int tc, auto BUF) {
    uint16_t* sb = decltype(BUF)::value ? sT1 : sT0;
    // 1 KB per wave and instruction; the image's last 2 KB go to waves 0 and 1
    const char* src = th + (size_t)tc * RT_BYTES;
#pragma unroll
    for (int i = 0; i < RT_BYTES / 4096; ++i)
      __builtin_amdgcn_global_load_lds((const glb_void_t*)(src + i * 4096),
                                       (lds_void_t*)((char*)sb + i * 4096 + wave * 1024), 16, 0, 0);
    if (wave < (RT_BYTES % 4096) / 1024)
      __builtin_amdgcn_global_load_lds((const glb_void_t*)(src + (RT_BYTES / 4096) * 4096),
                                       (lds_void_t*)((char*)sb + (RT_BYTES / 4096) * 4096 + wave * 1024),
                                       16, 0, 0);
  };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  issue(0, B0{});
#pragma unroll
  for (int i = 0; i < TA_CK / 256; ++i) {
    const int c = tid + 256 * i;
    const int pos = (c & ~31) + 16 * ((c >> 2) & 1) + 4 * ((c >> 3) & 3) + (c & 3);
    sCnt[pos] = F16T::from_f((float)kcounts[(size_t)h * TA_CK + c]);
  }
  if (tid < 64) sMask[tid] = (((tid >> 2) >> (tid & 3)) & 1) ? -__builtin_inff() : 0.f;
  uint32_t uw0 = ur[0], uw1 = ur[1];
  const float L2E = 1.4426950408889634f;
  float m2 = -1.0e30f, phi = 0.f;
  f32x16 O[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) O[nb] = zero16();
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // accumulator input of a half's score MFMA: nibble j of the lane's union
  // bits (elements 4 j .. 4 j + 3; element a <-> bit 8 (a / 4) + a % 4 after
  // the shift by 4 hh) selects a row of sMask, 0 or -inf
  auto mask_init = [&](uint32_t uword) {
    const uint32_t u4 = ((uword >> (4 * hh)) << 4) & 0xf0f0f0f0u;
    f32x16 S;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 mv = *(const f32x4*)((const char*)sMask + ((u4 >> (8 * j)) & 0xffu));
#pragma unroll
      for (int e = 0; e < 4; ++e) S[4 * j + e] = mv[e];
    }
    return S;
  };
  f32x16 Snext = mask_init(uw0);
  auto body = [&](int tc, auto BUF) {
    constexpr int buf = decltype(BUF)::value;
    const uint16_t* sb = buf ? sT1 : sT0;
    if (tc + 1 < RT_TILES) issue(tc + 1, std::integral_constant<int, buf ^ 1>{});
    uint32_t nw0 = 0, nw1 = 0;
    if (tc + 1 < RT_TILES) {
      nw0 = ur[2 * tc + 2];
      nw1 = ur[2 * tc + 3];
    }
    // per 32-centroid half kb: scores of the lane's query against centroids
    // 32 kb + 8 (a / 4) + 4 hh + a % 4 (element a of S), the union's
    // centroids at -inf; then the exponentials and P V of the half.  Working
    // a half at a time keeps the live scores and P fragments small.
    const uint16_t* vt = sb + 2048;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int r = 32 * kb + jl;
      // the union mask enters as the score MFMA's accumulator input, loaded
      // one half ahead
      f32x16 S = Snext;
      Snext = mask_init(kb ? nw0 : uw1);
      const u32x4 ca0 = *(const u32x4*)(sb + rc_off(r, hh));
      const u32x4 ca1 = *(const u32x4*)(sb + rc_off(r, 2 + hh));
      S = Mfma<F16T>::run(ca0, qu0, S);
      S = Mfma<F16T>::run(ca1, qu1, S);
      // fp16 scores (the reference rounds each centroid score to fp16), the
      // masked ones still -inf
      f16x2 sp[8];
#pragma unroll
      for (int a = 0; a < 16; a += 2)
        sp[a / 2] = __builtin_bit_cast(f16x2, Pk<F16T>::pack(S[a], S[a + 1]));
      // weights against the current max, without taking this half's max: the
      // exponentials scale exactly, so m2 only has to keep the fp16 P in
      // range.  The count-weighted sum of the half bounds the weight of every
      // cluster holding keys, and a weight that overflows to inf makes it inf
      // or (count 0) NaN; a half whose sum is not <= 2^14 (the first one,
      // m2 = -1e30, or scores far above the earlier ones) is redone with m2
      // moved past its max (the reference's lazy max), the sums so far
      // rescaled.  An empty cluster's weight can pass unseen only while finite.
      // The exponent argument reads the fp16 halves directly (v_fma_mix_f32).
      u32x4 pb[2];
      const u32x4* cw = (const u32x4*)(sCnt + TL_CT * tc + 32 * kb + 16 * hh);
      const u32x4 cn0 = cw[0], cn1 = cw[1];
      auto expo = [&](float nm) {
        float ph = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float pe[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            pe[e] = __builtin_amdgcn_exp2f(fmaf((float)sp[2 * j + e / 2][e % 2], L2E, nm));
          const uint32_t p01 = Pk<F16T>::pack(pe[0], pe[1]), p23 = Pk<F16T>::pack(pe[2], pe[3]);
          pb[j / 2][2 * (j % 2)] = p01;
          pb[j / 2][2 * (j % 2) + 1] = p23;
          // (copied to scalars first: a bit_cast straight from a vector element
          // reads element 0)
          const uint32_t c01 = (j < 2 ? cn0 : cn1)[2 * (j % 2)];
          const uint32_t c23 = (j < 2 ? cn0 : cn1)[2 * (j % 2) + 1];
          ph = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p01), __builtin_bit_cast(f16x2, c01),
                                      ph, false);
          ph = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p23), __builtin_bit_cast(f16x2, c23),
                                      ph, false);
        }
        return ph;
      };
      float pt = expo(-m2 * L2E);
      if (__builtin_amdgcn_readfirstlane((int)(__ballot(!(pt <= 0x1p14f)) != 0ull))) {
        T2T_REAL_BRANCH();
        f16x2 mp = {(_Float16)-__builtin_inff(), (_Float16)-__builtin_inff()};
#pragma unroll
        for (int a = 0; a < 8; ++a) mp = __builtin_elementwise_maximum(mp, sp[a]);
        float mx = vmax((float)mp[0], (float)mp[1]);
        mx = half_max(mx);
        const float mnew = mx > m2 ? mx + TL_MARGIN : m2;
        const float alpha = __builtin_amdgcn_exp2f((m2 - mnew) * L2E);
        m2 = mnew;
        phi *= alpha;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
          for (int a = 0; a < 16; ++a) O[nb][a] *= alpha;
        pt = expo(-m2 * L2E);
      }
      phi += pt;
      // the eight V^T fragments of the half are read together, so their LDS
      // latency is paid once rather than before every MFMA
      u32x4 vf[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        vf[i] = *(const u32x4*)(vt + vt_unit_off(32 * (i >> 1) + jl, 2 * (2 * kb + (i & 1)) + hh));
#pragma unroll
      for (int i = 0; i < 8; ++i) O[i >> 1] = Mfma<F16T>::run(vf[i], pb[i & 1], O[i >> 1]);
    }
    uw0 = nw0;
    uw1 = nw1;
    __builtin_amdgcn_s_waitcnt(0);  // tile tc + 1 landed
    __syncthreads();
  };
  for (int tc = 0; tc < RT_TILES; tc += 2) {
    body(tc, B0{});
    body(tc + 1, B1{});
  }
  if (!ok) return;
  // ---- merge under one softmax
  phi = half_sum(phi);
  const float tw = *tailw;
  const float lm = lam[h];
  const float le = lse2v[(size_t)h * N + row] * 0.6931471805599453f;
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
  // out row n of head h at out + h soh + n son (elements)
  uint16_t* orow = out + (size_t)h * soh + (size_t)orig * son;
  const uint16_t* er = SRC_SORTED ? exact + ((size_t)h * N + row) * TA_D : orow;
  if (bad && !SRC_SORTED) return;  // the exact part in out is the output
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * nb + 8 * g + 4 * hh;
      u32x2 v = *(const u32x2*)(er + d0);
      if (!bad) {
        const float x0 = T::to_f((uint16_t)(v[0] & 0xffff)), x1 = T::to_f((uint16_t)(v[0] >> 16));
        const float x2 = T::to_f((uint16_t)(v[1] & 0xffff)), x3 = T::to_f((uint16_t)(v[1] >> 16));
        v[0] = Pk<T>::pack(fmaf(wt, O[nb][4 * g], wx * x0), fmaf(wt, O[nb][4 * g + 1], wx * x1));
        v[1] = Pk<T>::pack(fmaf(wt, O[nb][4 * g + 2], wx * x2), fmaf(wt, O[nb][4 * g + 3], wx * x3));
      }
      *(u32x2*)(orow + d0) = v;
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
  T2T_REQUIRE(H > 0 && N > 0 && N < (1 << 24) && CQ > 0, "tile_attn_exact: H=%d N=%d CQ=%d", H, N, CQ);
  PlanView p = plan_view((int32_t*)plan, H, N, CQ);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == T2T_F16)
    launch_attn<F16T, 0>(q, kp, vp, unip, qperm, kcounts, p, attn_out, lse, nullptr, H, N, CQ, st);
  else
    launch_attn<BF16T, 0>(q, kp, vp, unip, qperm, kcounts, p, attn_out, lse, nullptr, H, N, CQ, st);
  T2T_LAUNCH_CHECK("tile_attn_exact");
  return T2T_OK;
}

extern "C" size_t t2t_centroid_tiles_bytes(int H) { return (size_t)H * RT_TILES * RT_BYTES; }

static void launch_centroid_tiles(const void* cks, const void* sumv, void* tiles, int H,
                                  hipStream_t st) {
  hipLaunchKernelGGL(centroid_tiles_kernel, dim3(RT_TILES, H), dim3(256), 0, st,
                     (const uint16_t*)cks, (const uint16_t*)sumv, (uint16_t*)tiles);
}

template <bool SRC_SORTED>
static void launch_resid(int dtype, const void* exact, const float* lse, const void* QU,
                         const void* tiles, const int32_t* kcounts, const int32_t* unip,
                         const int32_t* qlab, const int32_t* qperm, const float* lam,
                         const float* tailw, void* out, int H, int N, int CQ, hipStream_t st,
                         long long soh = -1, long long son = TA_D) {
  const dim3 grid(cdiv(N, 128), H);
  if (soh < 0) soh = (long long)N * TA_D;
  if (dtype == T2T_F16)
    hipLaunchKernelGGL((resid_kernel<F16T, SRC_SORTED>), grid, dim3(256), 0, st,
                       (const uint16_t*)exact, lse, (const uint16_t*)QU, (const uint16_t*)tiles,
                       kcounts, (const uint32_t*)unip, qlab, qperm, lam, tailw, (uint16_t*)out, N,
                       CQ, soh, son);
  else
    hipLaunchKernelGGL((resid_kernel<BF16T, SRC_SORTED>), grid, dim3(256), 0, st,
                       (const uint16_t*)exact, lse, (const uint16_t*)QU, (const uint16_t*)tiles,
                       kcounts, (const uint32_t*)unip, qlab, qperm, lam, tailw, (uint16_t*)out, N,
                       CQ, soh, son);
}

extern "C" size_t t2t_tail_merge_ws_bytes(int H) { return t2t_centroid_tiles_bytes(H); }

extern "C" int t2t_tail_merge(const void* attn_out, const float* lse, const void* QU,
                              const void* cks, const void* sumv, const int32_t* kcounts,
                              const int32_t* unip, const int32_t* qlab, const int32_t* qperm,
                              const float* lam, const float* tailw_dev, void* out, int dtype, int H,
                              int N, int CQ, void* ws, size_t ws_bytes, void* stream) {
  T2T_REQUIRE(attn_out && lse && QU && cks && sumv && kcounts && unip && qlab && qperm && lam &&
                  tailw_dev && out,
              "tail_merge: null pointer");
  T2T_REQUIRE(check_dtype(dtype), "tail_merge: dtype %d", dtype);
  T2T_REQUIRE(H > 0 && N > 0 && CQ > 0, "tail_merge: H=%d N=%d CQ=%d", H, N, CQ);
  if (!ws || ws_bytes < t2t_tail_merge_ws_bytes(H)) {
    t2t_set_error("tail_merge: workspace of %zu bytes, need %zu", ws_bytes,
                  t2t_tail_merge_ws_bytes(H));
    return T2T_ERR_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  launch_centroid_tiles(cks, sumv, ws, H, st);
  launch_resid<true>(dtype, attn_out, lse, QU, ws, kcounts, unip, qlab, qperm, lam, tailw_dev, out,
                     H, N, CQ, st);
  T2T_LAUNCH_CHECK("tail_merge");
  return T2T_OK;
}

extern "C" int t2t_centroid_tiles(const void* cks, const void* sumv, void* tiles, int H,
                                  void* stream) {
  T2T_REQUIRE(cks && sumv && tiles, "centroid_tiles: null pointer");
  T2T_REQUIRE(H > 0, "centroid_tiles: H=%d", H);
  launch_centroid_tiles(cks, sumv, tiles, H, (hipStream_t)stream);
  T2T_LAUNCH_CHECK("centroid_tiles");
  return T2T_OK;
}

static int exact_gather_impl(const void* q, long long sqh, long long sqn, const void* k,
                             long long skh, long long skn, const int32_t* kperm, const void* vp,
                             int dtype, const int32_t* kcounts, const int32_t* unip,
                             const int32_t* qperm, const int32_t* plan, void* out, long long soh,
                             long long son, float* lse, int H, int N, int CQ, void* stream) {
  T2T_REQUIRE(q && k && kperm && vp && kcounts && unip && qperm && plan && out && lse,
              "tile_attn_exact_orig_gather: null pointer");
  T2T_REQUIRE(check_dtype(dtype), "tile_attn_exact_orig_gather: dtype %d", dtype);
  T2T_REQUIRE(H > 0 && N > 0 && N < (1 << 24) && CQ > 0,
              "tile_attn_exact_orig_gather: H=%d N=%d CQ=%d", H, N, CQ);
  T2T_REQUIRE(sqn >= TA_D && skn >= TA_D && son >= TA_D && sqn % 8 == 0 && skn % 8 == 0 &&
                  son % 8 == 0 && sqh >= 0 && skh >= 0 && soh >= 0 && sqh % 8 == 0 &&
                  skh % 8 == 0 && soh % 8 == 0,
              "tile_attn_exact_orig_gather: strides must be non-negative multiples of 8 elements "
              "with row strides >= 128");
  T2T_REQUIRE((unsigned long long)(N - 1) * (unsigned long long)skn * 2ull + 256ull <= 0xFFFFFFFFull,
              "tile_attn_exact_orig_gather: one head's K rows span (N - 1) * %lld elements, more "
              "than 4 GiB", skn);
  PlanView p = plan_view((int32_t*)plan, H, N, CQ);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == T2T_F16)
    launch_attn<F16T, 2>(q, k, vp, unip, qperm, kcounts, p, nullptr, lse, out, H, N, CQ, st, kperm,
                         sqh, sqn, skh, skn, soh, son);
  else
    launch_attn<BF16T, 2>(q, k, vp, unip, qperm, kcounts, p, nullptr, lse, out, H, N, CQ, st, kperm,
                          sqh, sqn, skh, skn, soh, son);
  T2T_LAUNCH_CHECK("tile_attn_exact_orig_gather");
  return T2T_OK;
}

extern "C" int t2t_tile_attn_exact_orig_gather(const void* q, const void* k, const int32_t* kperm,
                                               const void* vp, int dtype, const int32_t* kcounts,
                                               const int32_t* unip, const int32_t* qperm,
                                               const int32_t* plan, void* out, float* lse, int H,
                                               int N, int CQ, void* stream) {
  const long long hs = (long long)N * TA_D;
  return exact_gather_impl(q, hs, TA_D, k, hs, TA_D, kperm, vp, dtype, kcounts, unip, qperm, plan,
                           out, hs, TA_D, lse, H, N, CQ, stream);
}

extern "C" int t2t_tile_attn_exact_orig_gather_strided(
    const void* q, long long q_head_stride, long long q_row_stride, const void* k,
    long long k_head_stride, long long k_row_stride, const int32_t* kperm, const void* vp,
    int dtype, const int32_t* kcounts, const int32_t* unip, const int32_t* qperm,
    const int32_t* plan, void* out, long long out_head_stride, long long out_row_stride,
    float* lse, int H, int N, int CQ, void* stream) {
  return exact_gather_impl(q, q_head_stride, q_row_stride, k, k_head_stride, k_row_stride, kperm,
                           vp, dtype, kcounts, unip, qperm, plan, out, out_head_stride,
                           out_row_stride, lse, H, N, CQ, stream);
}

extern "C" int t2t_tile_attn_exact_orig_gather_kv_strided(
    const void* q, long long q_head_stride, long long q_row_stride, const void* k,
    long long k_head_stride, long long k_row_stride, const void* v, long long v_head_stride,
    long long v_row_stride, const int32_t* kperm, int dtype, const int32_t* kcounts,
    const int32_t* unip, const int32_t* qperm, const int32_t* plan, void* out,
    long long out_head_stride, long long out_row_stride, float* lse, int H, int N, int CQ,
    void* stream) {
  T2T_REQUIRE(q && k && v && kperm && kcounts && unip && qperm && plan && out && lse,
              "tile_attn_exact_orig_gather_kv: null pointer");
  T2T_REQUIRE(check_dtype(dtype), "tile_attn_exact_orig_gather_kv: dtype %d", dtype);
  T2T_REQUIRE(H > 0 && N > 0 && N < (1 << 24) && CQ > 0,
              "tile_attn_exact_orig_gather_kv: H=%d N=%d CQ=%d", H, N, CQ);
  const long long st4[8] = {q_head_stride, q_row_stride, k_head_stride, k_row_stride,
                            v_head_stride, v_row_stride, out_head_stride, out_row_stride};
  for (int i = 0; i < 8; ++i)
    T2T_REQUIRE(st4[i] >= 0 && st4[i] % 8 == 0 && (i % 2 == 0 || st4[i] >= TA_D),
                "tile_attn_exact_orig_gather_kv: strides must be non-negative multiples of 8 "
                "elements with row strides >= 128");
  for (long long rs : {k_row_stride, v_row_stride})
    T2T_REQUIRE((unsigned long long)(N - 1) * (unsigned long long)rs * 2ull + 256ull <= 0xFFFFFFFFull,
                "tile_attn_exact_orig_gather_kv: one head's K or V rows span (N - 1) * %lld "
                "elements, more than 4 GiB", rs);
  PlanView p = plan_view((int32_t*)plan, H, N, CQ);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == T2T_F16)
    launch_attn<F16T, 3>(q, k, v, unip, qperm, kcounts, p, nullptr, lse, out, H, N, CQ, st, kperm,
                         q_head_stride, q_row_stride, k_head_stride, k_row_stride, out_head_stride,
                         out_row_stride, v_head_stride, v_row_stride);
  else
    launch_attn<BF16T, 3>(q, k, v, unip, qperm, kcounts, p, nullptr, lse, out, H, N, CQ, st, kperm,
                          q_head_stride, q_row_stride, k_head_stride, k_row_stride,
                          out_head_stride, out_row_stride, v_head_stride, v_row_stride);
  T2T_LAUNCH_CHECK("tile_attn_exact_orig_gather_kv");
  return T2T_OK;
}

extern "C" int t2t_tile_attn_exact_orig(const void* q, const void* kp, const void* vp, int dtype,
                                        const int32_t* kcounts, const int32_t* unip,
                                        const int32_t* qperm, const int32_t* plan, void* out,
                                        float* lse, int H, int N, int CQ, void* stream) {
  T2T_REQUIRE(q && kp && vp && kcounts && unip && qperm && plan && out && lse,
              "tile_attn_exact_orig: null pointer");
  T2T_REQUIRE(check_dtype(dtype), "tile_attn_exact_orig: dtype %d", dtype);
  T2T_REQUIRE(H > 0 && N > 0 && N < (1 << 24) && CQ > 0, "tile_attn_exact_orig: H=%d N=%d CQ=%d",
              H, N, CQ);
  PlanView p = plan_view((int32_t*)plan, H, N, CQ);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == T2T_F16)
    launch_attn<F16T, 1>(q, kp, vp, unip, qperm, kcounts, p, nullptr, lse, out, H, N, CQ, st);
  else
    launch_attn<BF16T, 1>(q, kp, vp, unip, qperm, kcounts, p, nullptr, lse, out, H, N, CQ, st);
  T2T_LAUNCH_CHECK("tile_attn_exact_orig");
  return T2T_OK;
}

static int resid_inplace_impl(void* out, long long soh, long long son, const float* lse,
                              const void* QU, const void* tiles, const int32_t* kcounts,
                              const int32_t* unip, const int32_t* qlab, const int32_t* qperm,
                              const float* lam, const float* tailw_dev, int dtype, int H, int N,
                              int CQ, void* stream) {
  T2T_REQUIRE(out && lse && QU && tiles && kcounts && unip && qlab && qperm && lam && tailw_dev,
              "resid_merge_inplace: null pointer");
  T2T_REQUIRE(check_dtype(dtype), "resid_merge_inplace: dtype %d", dtype);
  T2T_REQUIRE(H > 0 && N > 0 && CQ > 0, "resid_merge_inplace: H=%d N=%d CQ=%d", H, N, CQ);
  T2T_REQUIRE(son >= TA_D && son % 8 == 0 && soh >= 0 && soh % 8 == 0,
              "resid_merge_inplace: out strides (%lld, %lld)", soh, son);
  launch_resid<false>(dtype, nullptr, lse, QU, tiles, kcounts, unip, qlab, qperm, lam, tailw_dev,
                      out, H, N, CQ, (hipStream_t)stream, soh, son);
  T2T_LAUNCH_CHECK("resid_merge_inplace");
  return T2T_OK;
}

extern "C" int t2t_resid_merge_inplace(void* out, const float* lse, const void* QU,
                                       const void* tiles, const int32_t* kcounts,
                                       const int32_t* unip, const int32_t* qlab,
                                       const int32_t* qperm, const float* lam,
                                       const float* tailw_dev, int dtype, int H, int N, int CQ,
                                       void* stream) {
  return resid_inplace_impl(out, (long long)N * TA_D, TA_D, lse, QU, tiles, kcounts, unip, qlab,
                            qperm, lam, tailw_dev, dtype, H, N, CQ, stream);
}

extern "C" int t2t_resid_merge_inplace_strided(void* out, long long out_head_stride,
                                               long long out_row_stride, const float* lse,
                                               const void* QU, const void* tiles,
                                               const int32_t* kcounts, const int32_t* unip,
                                               const int32_t* qlab, const int32_t* qperm,
                                               const float* lam, const float* tailw_dev,
                                               int dtype, int H, int N, int CQ, void* stream) {
  return resid_inplace_impl(out, out_head_stride, out_row_stride, lse, QU, tiles, kcounts, unip,
                            qlab, qperm, lam, tailw_dev, dtype, H, N, CQ, stream);
}

extern "C" size_t t2t_tile_attn_ws_bytes(int H, int N, int dtype) {
  (void)dtype;
  return t2t_align256((size_t)H * N * sizeof(float)) + t2t_centroid_tiles_bytes(H);
}

extern "C" int t2t_tile_attn_run_planned(const void* q, const void* kp, const void* vp, int dtype,
                                         const int32_t* qcounts, const int32_t* kcounts,
                                         const int32_t* unip, const void* QU, const void* cks,
                                         const void* sumv, const float* lam, const int32_t* qlab,
                                         const int32_t* qperm, const float* tailw_dev, void* out,
                                         int32_t* plan, int rebuild_plan, int H, int N, int CQ,
                                         void* ws, size_t ws_bytes, void* stream) {
  T2T_REQUIRE(q && kp && vp && qcounts && kcounts && unip && QU && cks && sumv && lam && qlab &&
                  qperm && tailw_dev && out && plan,
              "tile_attn_run_planned: null pointer");
  T2T_REQUIRE(check_dtype(dtype), "tile_attn_run_planned: dtype %d", dtype);
  T2T_REQUIRE(H > 0 && N > 0 && N < (1 << 24) && CQ > 0, "tile_attn_run_planned: H=%d N=%d CQ=%d", H, N, CQ);
  hipStream_t st = (hipStream_t)stream;
  if (rebuild_plan) {
    const int rc = t2t_tile_plan(qcounts, kcounts, unip, plan, H, N, CQ, stream);
    if (rc) return rc;
  }
  const size_t need = t2t_tile_attn_ws_bytes(H, N, dtype);
  if (!ws || ws_bytes < need) {
    t2t_set_error("tile_attn_run_planned: workspace of %zu bytes, need %zu", ws_bytes, need);
    return T2T_ERR_WORKSPACE;
  }
  float* lse = (float*)ws;
  void* tiles = (char*)ws + t2t_align256((size_t)H * N * sizeof(float));
  PlanView p = plan_view(plan, H, N, CQ);
  launch_centroid_tiles(cks, sumv, tiles, H, st);
  if (dtype == T2T_F16)
    launch_attn<F16T, 1>(q, kp, vp, unip, qperm, kcounts, p, nullptr, lse, out, H, N, CQ, st);
  else
    launch_attn<BF16T, 1>(q, kp, vp, unip, qperm, kcounts, p, nullptr, lse, out, H, N, CQ, st);
  launch_resid<false>(dtype, nullptr, lse, QU, tiles, kcounts, unip, qlab, qperm, lam, tailw_dev,
                      out, H, N, CQ, st);
  T2T_LAUNCH_CHECK("tile_attn_run_planned");
  return T2T_OK;
}
