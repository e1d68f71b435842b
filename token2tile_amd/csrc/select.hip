// S4: per-query key-cluster selection and query-cluster union (gfx950).
//
// One wave owns a run of consecutive SORTED query rows (qperm order), so the
// work is balanced whatever the query-cluster sizes are.  (The fused scoring
// + selection kernel below first tries a one-pass window around the previous
// row's crossing key, which resolves nearly every row; the radix passes
// described here are its fallback and the unfused kernel's method.)  For each row the
// 2048 fp16 scores sit in registers (lane l holds clusters 512 g + 8 l + j,
// g < 4, j < 8), and the budget threshold is found exactly with two 8-bit
// radix passes over a wave-private, size-weighted LDS histogram:
//   pass 1: high byte of the ordered key, pass 2: low byte inside the
//   crossing high-byte bin.  Only keys above a lower bound carried over from
//   the previous row enter the histogram (exact: a row whose bounded keys do
//   not reach the budget is redone without the bound).
// Ties at the threshold are resolved in ascending cluster order with wave
// prefix sums.  Each lane keeps the OR of its 32 selection bits across the
// rows of one query cluster and flushes them with one atomicOr per word when
// the run crosses into the next cluster, so the union needs no partial
// buffers.
#include "t2t_common.h"
#include <mutex>

#define SEL_NC 2048
#define SEL_WAVES 4
#define SEL_ROWS_PER_WAVE 16
// per-wave histogram: 256 bins plus one private dump slot per lane, so both
// passes add every key without a branch (pass 2 sends keys outside the
// crossing high-byte bin to the lane's own slot: no conflicts, never read)
#define SEL_HIST (256 + 64)

// compiler-only ordering of LDS accesses (no wait): for wave-private LDS
// data, whose accesses the wave's LDS queue performs in issue order
__device__ inline void lds_order() { asm volatile("" ::: "memory"); }

#define SEL_CAND1 4  // window candidates per lane in the first round of LDS reads
#define SEL_CAND 4   // ... and in each further round

__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// off[h, 0..CQ] = exclusive scan of qcounts (off[CQ] = total rows); zero unip
__global__ __launch_bounds__(1024) void select_prep_kernel(const int32_t* __restrict__ qcounts,
                                                           int32_t* __restrict__ off,
                                                           int32_t* __restrict__ unip, int CQ) {
  __shared__ int wsum[16];
  __shared__ int carry;
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int c0 = 0; c0 < CQ; c0 += 1024) {
    const int c = c0 + tid;
    const int v = c < CQ ? qcounts[(size_t)h * CQ + c] : 0;
    const int inc = wave_incl_scan(v);
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    int add = carry;
    for (int i = 0; i < w; ++i) add += wsum[i];
    if (c < CQ) off[(size_t)h * (CQ + 1) + c] = add + inc - v;
    __syncthreads();
    if (tid == 1023) carry = add + inc;
    __syncthreads();
  }
  if (tid == 0) off[(size_t)h * (CQ + 1) + CQ] = carry;
  int32_t* u = unip + (size_t)h * CQ * (SEL_NC / 32);
  for (int i = tid; i < CQ * (SEL_NC / 32); i += 1024) u[i] = 0;
}

// Find the bin where the running (descending) weight first reaches ns.
// hist has 256 bins, bin 255 = largest keys.  Lane l scans bins 255-4l..252-4l.
// Returns the bin; *above = weight of all higher bins; *inbin = its weight;
// *total = base + the weight of all bins (below ns: no bin crosses and the
// returned bin is meaningless).
// PACKED: the bins hold (weight << 12) | key count; *count = the crossing
// bin's key count (unused otherwise).
template <bool PACKED = false>
__device__ inline int find_cross(const int* hist, int base, int ns, int* above, int* inbin,
                                 int* total, int* count = nullptr) {
  const int l = __lane_id();
  int w[4], cn[4];
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int raw = hist[255 - 4 * l - i];
    w[i] = PACKED ? raw >> 12 : raw;
    cn[i] = raw & 0xfff;
    s += w[i];
  }
  const int inc = wave_incl_scan(s);
  const int ex = inc - s + base;
  *total = base + __builtin_amdgcn_readlane(inc, 63);
  const bool mine = (ex < ns) && (ex + s >= ns);
  int bin = 0, ab = 0, ib = 0, ic = 0;
  if (mine) {
    int cum = ex;
    bool done = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!done && cum + w[i] >= ns) {
        bin = 255 - 4 * l - i;
        ab = cum;
        ib = w[i];
        ic = cn[i];
        done = true;
      }
      cum += w[i];
    }
  }
  const unsigned long long bal = __ballot(mine);
  const int src = bal ? (int)__ffsll((long long)bal) - 1 : 0;
  *above = __builtin_amdgcn_readlane(ab, src);
  *inbin = __builtin_amdgcn_readlane(ib, src);
  if (PACKED) *count = __builtin_amdgcn_readlane(ic, src);
  return __builtin_amdgcn_readlane(bin, src);
}

// the order keys of a pair of fp16 scores (score_key on each half): the sign
// of each half spread over it (v_pk_ashrrev_i16), then x ^ (sign & 0x7FFF)
// per half in one three-input bit operation
typedef short s16x2 __attribute__((ext_vector_type(2)));
__device__ inline uint32_t key_pair(uint32_t x) {
  const uint32_t sm = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s16x2, x) >> (s16x2){15, 15});
  return x ^ (sm & 0x7FFF7FFFu);
}

// The lane's 32 order keys stay packed two to a dword as they sit in the
// score row: slot i (cluster 512 (i / 8) + 8 lane + i % 8) is the low (i even)
// or high (i odd) half of kp[i / 2].
// cluster of slot i of lane l
__device__ inline int slot_cluster(int i, int l) { return 512 * (i >> 3) + 8 * l + (i & 7); }
// column of cluster c in a staged key row whose 16-byte chunks are XOR
// swizzled by rsw (the row index mod 16)
__device__ inline int key_col(int c, int rsw) { return 8 * ((c >> 3) ^ rsw) + (c & 7); }
__device__ inline int key_at(const uint32_t (&kp)[16], int i) {
  return (int)(int16_t)(uint16_t)((i & 1) ? kp[i >> 1] >> 16 : kp[i >> 1] & 0xffffu);
}
// bit i = (key i OP t), OP = ge / gt / eq: one compare per key on its
// sign-extended half (SDWA) into VCC, then m + m + carry, from slot 31 down
#define KEY_MASK_STEP(CMP, SEL)                                                        \
  asm("v_cmp_" CMP "_i32_sdwa vcc, sext(%1), %2 src0_sel:" SEL " src1_sel:DWORD\n\t" \
      "v_addc_co_u32 %0, vcc, %0, %0, vcc"                                            \
      : "+v"(m)                                                                        \
      : "v"(kp[i >> 1]), "v"(t)                                                        \
      : "vcc")
#define KEY_MASK_BODY(CMP)                                        \
  uint32_t m = 0;                                                 \
  _Pragma("unroll") for (int i = 31; i >= 0; --i) {               \
    if (i & 1) KEY_MASK_STEP(CMP, "WORD_1"); else KEY_MASK_STEP(CMP, "WORD_0"); \
  }                                                               \
  return m;
__device__ inline uint32_t keys_ge(const uint32_t (&kp)[16], int t) { KEY_MASK_BODY("ge") }
__device__ inline uint32_t keys_gt(const uint32_t (&kp)[16], int t) { KEY_MASK_BODY("gt") }
__device__ inline uint32_t keys_eq(const uint32_t (&kp)[16], int t) { KEY_MASK_BODY("eq") }

// Selection of one row.  kp: the lane's 32 clusters (index 8 g + j); ssz: the
// head's cluster sizes (LDS).
// Returns the lane's 32 selection bits; *rowcnt = selected keys (all lanes);
// *vstar_out = the row's crossing key.
//
// lo (wave-uniform) is a guess for a lower bound of the crossing key: the
// previous row's crossing key minus SEL_BOUND_MARGIN, or SEL_NO_BOUND.  Keys
// below it go to the lane's private dump slot instead of a histogram bin,
// which removes the bulk of a row's keys (similar scores share a few high-byte
// bins) from the same-address atomic conflicts.  The result is exact whenever
// the clusters with keys >= lo hold >= ns keys: the crossing key is then >= lo
// and every key at or above it is counted.  Otherwise the row is redone
// without the bound.
__device__ inline uint32_t select_bits(const uint32_t (&kp)[16], const int* ssz, int ns, int vstar,
                                       int wgt, int weq, int ntie, int* rowcnt);
#define SEL_NO_BOUND (-65536)
#define SEL_BOUND_MARGIN 1024  // one binade of fp16 keys
__device__ inline void radix_cross(const uint32_t (&kp)[16], const int* ssz, int* hist, int ns,
                                   int lo, int* vstar_out, int* wgt_out, int* weq_out,
                                   int* ntie_out) {
  const int l = __lane_id();
  // ---- pass 1: high byte ----
  int hb, above1, inbin1, tot1;
  for (;;) {
#pragma unroll
    for (int i = 0; i < 4; ++i) hist[4 * l + i] = 0;
    wave_sync();
#pragma unroll
    for (int i = 0; i < 32; ++i) {  // empty clusters add 0
      const int key = key_at(kp, i);
      atomicAdd(&hist[key >= lo ? (key >> 8) + 128 : 256 + l], ssz[slot_cluster(i, l)]);
    }
    wave_sync();
    hb = find_cross(hist, 0, ns, &above1, &inbin1, &tot1);
    wave_sync();
    if (tot1 >= ns || lo == SEL_NO_BOUND) break;  // wave-uniform
    lo = SEL_NO_BOUND;
  }
  // ---- pass 2: low byte within the crossing high-byte bin ----
#pragma unroll
  for (int i = 0; i < 4; ++i) hist[4 * l + i] = 0;
  wave_sync();
  const int hsel = hb - 128;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int key = key_at(kp, i);
    atomicAdd(&hist[(key >> 8) == hsel && key >= lo ? (key & 255) : 256 + l],
              (ssz[slot_cluster(i, l)] << 12) | 1);  // weight and key count (weights < 2^19, counts < 2^12)
  }
  wave_sync();
  int wgt, weq, tot2, ntie;
  const int lb = find_cross<true>(hist, above1, ns, &wgt, &weq, &tot2, &ntie);
  wave_sync();
  *vstar_out = hsel * 256 + lb;
  *wgt_out = wgt;
  *weq_out = weq;
  *ntie_out = ntie;
}
__device__ inline uint32_t select_row(const uint32_t (&kp)[16], const int* ssz, int* hist, int ns,
                                      int lo, int* rowcnt, int* vstar_out) {
  int wgt, weq, ntie;
  radix_cross(kp, ssz, hist, ns, lo, vstar_out, &wgt, &weq, &ntie);
  return select_bits(kp, ssz, ns, *vstar_out, wgt, weq, ntie, rowcnt);
}

// The lane's 32 selection bits given the crossing key vstar of the row, the
// weight wgt of all keys above it, the weight weq and number ntie of the
// clusters holding vstar; *rowcnt = selected keys.  Ties at the threshold
// (ntie > 1) are taken in ascending cluster order.
__device__ inline uint32_t select_bits(const uint32_t (&kp)[16], const int* ssz, int ns, int vstar,
                                       int wgt, int weq, int ntie, int* rowcnt) {
  const int l = __lane_id();
  if (ntie == 1) {
    *rowcnt = wgt + weq;
    return keys_ge(kp, vstar);
  }
  // ---- several clusters on the key vstar: all keys above it are taken
  //      (weight wgt < ns), then the tied clusters in ascending cluster order
  //      (index 512 g + 8 lane + j) until their weight reaches R; the tied
  //      cluster where it does is istar, and every tied cluster up to it is
  //      taken, empty ones included
  const int R = ns - wgt;  // >= 1
  const uint32_t gt = keys_gt(kp, vstar), tie = keys_eq(kp, vstar);
  int cum = 0, istar = -1;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    unsigned long long bal = __ballot(((tie >> (8 * g)) & 0xffu) != 0u);
    while (bal != 0ull && istar < 0) {  // wave-uniform
      const int L = (int)__ffsll((long long)bal) - 1;
      bal &= bal - 1ull;
      const uint32_t byte = ((uint32_t)__builtin_amdgcn_readlane((int)tie, L) >> (8 * g)) & 0xffu;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (istar < 0 && ((byte >> j) & 1u)) {
          cum += ssz[512 * g + 8 * L + j];
          if (cum >= R) istar = 512 * g + 8 * L + j;
        }
      }
    }
  }
  // tied keys of the lane with cluster index <= istar
  uint32_t upto = 0;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    int w = istar - (512 * g + 8 * l) + 1;
    w = w < 0 ? 0 : (w > 8 ? 8 : w);
    upto |= ((1u << w) - 1u) << (8 * g);
  }
  *rowcnt = wgt + cum;
  return gt | (tie & upto);
}

// Single-pass crossing search in a window of SEL_WIN consecutive keys [lo,
// lo + SEL_WIN) placed around the previous row's crossing key.  Only the lane's keys
// at or above lo are visited (a few per lane): a key in the window adds
// (size << 12) | 1 to its own bin of a wave-private LDS histogram, a key above
// it adds its size to a register sum; keys below lo are not touched.  The
// bins then hold the exact weight and cluster count of every key value in the
// window, and the sum the weight above it.  When the crossing lies in the
// window (weight above < ns <= weight above + window weight) this gives the
// crossing key, the weight above it and the weight and count of its clusters
// without the two radix passes (returns 0); otherwise it returns 1 (crossing
// above the window) or -1 (below it).
#define SEL_WIN 448
#define SEL_WPL (SEL_WIN / 64)  // window bins per lane
#define SEL_WHIST SEL_WIN  // window bins (the radix fallback uses the first 320)
__device__ inline int window_cross(const uint32_t (&kp)[16], const uint16_t* krow, int rsw, const int* ssz,
                                   int* hist, int ns, int lo, int* vstar, int* wgt, int* weq,
                                   int* ntie, uint32_t* bits, int* bits_ok) {
  const int l = __lane_id();
  // The histogram is private to the wave, and a wave's LDS instructions are
  // performed in the order it issues them, so the clear, the adds and the
  // reads below need no memory wait between them: the compiler barriers
  // (lds_order) only keep the compiler from reordering them.
#pragma unroll
  for (int i = 0; i < (SEL_WIN + 255) / 256; ++i)
    if (l + 64 * i < SEL_WIN / 4) *(u32x4*)(hist + 4 * (l + 64 * i)) = u32x4{0u, 0u, 0u, 0u};
  lds_order();
  // the lane's keys at or above the window's base, as a mask
  uint32_t m = keys_ge(kp, lo);
  int aw = 0;  // the lane's weight above the window
  // candidates in rounds per lane: a round's key and size reads are issued
  // together (one LDS latency per round, not per key); a lane with fewer
  // candidates reads cluster 0 for the rest and adds nothing.  The first
  // round takes SEL_CAND1 and keeps their slots and keys, which give the
  // selection bits directly when it was the only round
  int slot1[SEL_CAND1], d1[SEL_CAND1];
  bool ok1[SEL_CAND1];
  {
    int c[SEL_CAND1], sz[SEL_CAND1];
#pragma unroll
    for (int it = 0; it < SEL_CAND1; ++it) {
      ok1[it] = m != 0u;
      slot1[it] = __builtin_ctz(m | 0x80000000u);
      m &= m - 1u;
      c[it] = ok1[it] ? slot_cluster(slot1[it], l) : 0;
    }
#pragma unroll
    for (int it = 0; it < SEL_CAND1; ++it) {
      d1[it] = (int)(int16_t)krow[key_col(c[it], rsw)] - lo;
      sz[it] = ssz[c[it]];
    }
#pragma unroll
    for (int it = 0; it < SEL_CAND1; ++it) {
      aw += ok1[it] && d1[it] >= SEL_WIN ? sz[it] : 0;
      if (ok1[it] && d1[it] < SEL_WIN) atomicAdd(&hist[d1[it]], (sz[it] << 12) | 1);
    }
  }
  const bool one_round = __ballot(m != 0u) == 0ull;  // wave-uniform
  while (__ballot(m != 0u) != 0ull) {  // wave-uniform
    int c[SEL_CAND];
    bool ok[SEL_CAND];
#pragma unroll
    for (int it = 0; it < SEL_CAND; ++it) {
      ok[it] = m != 0u;
      const int i = __builtin_ctz(m | 0x80000000u);
      m &= m - 1u;
      c[it] = ok[it] ? slot_cluster(i, l) : 0;
    }
    int d[SEL_CAND], sz[SEL_CAND];
#pragma unroll
    for (int it = 0; it < SEL_CAND; ++it) {
      d[it] = (int)(int16_t)krow[key_col(c[it], rsw)] - lo;
      sz[it] = ssz[c[it]];
    }
#pragma unroll
    for (int it = 0; it < SEL_CAND; ++it) {
      aw += ok[it] && d[it] >= SEL_WIN ? sz[it] : 0;
      if (ok[it] && d[it] < SEL_WIN) atomicAdd(&hist[d[it]], (sz[it] << 12) | 1);
    }
  }
  lds_order();
  // lane l scans its SEL_WPL bins, from the top (descending keys)
  int raw[SEL_WPL];
  int s = 0;
#pragma unroll
  for (int i = 0; i < SEL_WPL; ++i) {
    raw[i] = hist[SEL_WIN - 1 - SEL_WPL * l - i];
    s += raw[i] >> 12;
  }
  const int above = wave_sum(aw);
  const int inc = wave_incl_scan(s);
  const int total = above + __builtin_amdgcn_readlane(inc, 63);
  lds_order();
  if (above >= ns) return 1;  // wave-uniform: the crossing is above the window
  if (total < ns) return -1;  // below it
  const int ex = inc - s + above;
  const bool mine = ex < ns && ex + s >= ns;
  int bin = 0, ab = 0, raw_b = 0;
  if (mine) {
    int cum = ex;
    bool done = false;
#pragma unroll
    for (int i = 0; i < SEL_WPL; ++i) {
      const int w = raw[i] >> 12;
      if (!done && cum + w >= ns) {
        bin = SEL_WIN - 1 - SEL_WPL * l - i;
        ab = cum;
        raw_b = raw[i];
        done = true;
      }
      cum += w;
    }
  }
  const unsigned long long bal = __ballot(mine);
  const int src = (int)__ffsll((long long)bal) - 1;
  *vstar = lo + __builtin_amdgcn_readlane(bin, src);
  *wgt = __builtin_amdgcn_readlane(ab, src);
  raw_b = __builtin_amdgcn_readlane(raw_b, src);
  *weq = raw_b >> 12;
  *ntie = raw_b & 0xfff;
  // one cluster at the crossing key: the selection is every key at or above
  // it, all of them candidates (keys >= lo); from the first round's records
  // when it held them all
  *bits_ok = one_round && *ntie == 1;
  if (*bits_ok) {
    const int t = *vstar - lo;
    uint32_t b = 0;
#pragma unroll
    for (int it = 0; it < SEL_CAND1; ++it) b |= ok1[it] && d1[it] >= t ? 1u << slot1[it] : 0u;
    *bits = b;
  }
  return 0;
}

// publish the lanes' masks into the packed union row (LSB-first words);
// must be called by the whole wave (it shuffles across lanes)
__device__ inline void flush_union(uint32_t acc, int32_t* urow) {
  const int l = __lane_id();
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t b = (acc >> (8 * g)) & 0xffu;
    // lanes 4q + 1 .. 4q + 3 of the quad (DPP quad_perm [1,1,1,1], [2,2,2,2], [3,3,3,3])
    const uint32_t b1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)b, 0x55, 0xf, 0xf, false);
    const uint32_t b2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)b, 0xaa, 0xf, 0xf, false);
    const uint32_t b3 = (uint32_t)__builtin_amdgcn_mov_dpp((int)b, 0xff, 0xf, 0xf, false);
    const uint32_t w = b | (b1 << 8) | (b2 << 16) | (b3 << 24);
    if ((l & 3) == 0 && w) atomicOr((unsigned int*)&urow[16 * g + (l >> 2)], w);
  }
}

__global__ __launch_bounds__(SEL_WAVES * 64) void select_main_kernel(
    const uint16_t* __restrict__ gl, const int32_t* __restrict__ kcounts,
    const int32_t* __restrict__ qperm, const int32_t* __restrict__ off,
    const int32_t* __restrict__ ns_dev, int32_t* __restrict__ unip, int32_t* __restrict__ rowcnt,
    int N, int CQ) {
  __shared__ int hist_all[SEL_WAVES][SEL_HIST];
  __shared__ int sSz[SEL_NC];  // the head's key-cluster sizes
  const int h = blockIdx.y;
  const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int* hist = hist_all[wv];
  for (int c = threadIdx.x; c < SEL_NC; c += SEL_WAVES * 64) sSz[c] = kcounts[(size_t)h * SEL_NC + c];
  __syncthreads();
  const int32_t* offh = off + (size_t)h * (CQ + 1);
  const int total = offh[CQ];
  int j0 = (blockIdx.x * SEL_WAVES + wv) * SEL_ROWS_PER_WAVE;
  int j1 = j0 + SEL_ROWS_PER_WAVE;
  if (j1 > total) j1 = total;
  if (j1 > N) j1 = N;  // qcounts summing past N is invalid input; never read past N
  if (j0 >= j1) return;
  // the key total
  int ktot = 0;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int32_t* p = kcounts + (size_t)h * SEL_NC + 512 * g + 8 * l;
#pragma unroll
    for (int j = 0; j < 8; ++j) ktot += p[j];
  }
  ktot = wave_sum(ktot);
  int ns = *ns_dev;
  ns = ns < 1 ? 1 : ns;
  ns = ns > ktot ? ktot : ns;
  // query cluster of the first row: largest t with off[t] <= j0
  int lo = 0, hi = CQ - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offh[mid] <= j0) lo = mid; else hi = mid - 1;
  }
  int t = lo;
  while (t < CQ - 1 && offh[t + 1] <= j0) ++t;  // skip empty clusters
  int tend = offh[t + 1];
  uint32_t acc = 0;
  int klo = SEL_NO_BOUND, vstar = 0;  // lower-bound guess from the previous row
  const uint16_t* glh = gl + (size_t)h * N * SEL_NC;
  const int32_t* qp = qperm + (size_t)h * N;
  int32_t* uh = unip + (size_t)h * CQ * (SEL_NC / 32);
  for (int j = j0; j < j1; ++j) {
    if (j >= tend) {  // wave-uniform: every lane takes part in the shuffles
      flush_union(acc, uh + (size_t)t * (SEL_NC / 32));
      acc = 0;
      do {
        ++t;
        tend = offh[t + 1];
      } while (j >= tend);
    }
    const int orig = qp[j];
    uint32_t kp[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u32x4 v = __builtin_nontemporal_load(
          (const u32x4*)(glh + (size_t)orig * SEL_NC + 512 * g + 8 * l));
#pragma unroll
      for (int q = 0; q < 4; ++q) kp[4 * g + q] = key_pair(v[q]);
    }
    int rc;
    acc |= select_row(kp, sSz, hist, ns, klo, &rc, &vstar);
    klo = vstar - SEL_BOUND_MARGIN;
    if (l == 0) rowcnt[(size_t)h * N + orig] = rc;
  }
  flush_union(acc, uh + (size_t)t * (SEL_NC / 32));
}

// ---------------------------------------------------------------------------
// Fused scoring + selection: the scores never leave the chip.  One 12-wave
// work-group per CU (three waves per SIMD) takes batches of 32 consecutive
// sorted rows: every wave computes the scores of the batch against 160 or 192
// of the centroids on MFMA, with
// the instruction, operand split and fp16 rounding of score_kernel (so the
// scores, and the selection, are bit-identical to the unfused path), and
// stores the ordered keys in LDS; then the waves select the rows, taking
// them one at a time from a counter.  A row is searched in a 448-key window
// around the previous row's crossing (window_cross: a few keys per lane, one
// histogram pass), then in the window above or below it, and by the radix
// passes only when both miss (a few rows in 10^4 at 720p).  A work-group
// walks 16 batches (512 rows): the cluster sizes it loads once are amortised
// over them, and the next batch's query rows load while the current batch is
// being selected.  LDS: the batch's keys (128 KB; 16-byte chunks XOR
// swizzled by row instead of padded), twelve 1.75 KB window histograms and the
// cluster sizes.  The centroid fragments are reloaded from L2 per batch (held
// across batches they would push the kernel past the 168 registers of three
// waves per SIMD), each wave issuing the next batch's loads just before the
// batch's closing barrier, so that their latency hides behind it.
// ---------------------------------------------------------------------------
#define SF_WAVES 12
#define SF_ROWS 32
#define SF_BATCHES 16
#define SF_PITCH SEL_NC  // halves per LDS key row (chunks swizzled by row, no padding)
#define SF_TILES 6       // most 32-centroid score tiles a wave holds (64 tiles over 12 waves)


__global__ __launch_bounds__(SF_WAVES * 64, 1) void score_select_kernel(
    const uint16_t* __restrict__ QU, const uint16_t* __restrict__ cks,
    const int32_t* __restrict__ kcounts, const int32_t* __restrict__ qperm,
    const int32_t* __restrict__ off, const int32_t* __restrict__ ns_dev,
    int32_t* __restrict__ unip, int32_t* __restrict__ rowcnt, int N, int CQ) {
  __shared__ __attribute__((aligned(16))) uint16_t sKey[SF_ROWS * SF_PITCH];
  __shared__ __attribute__((aligned(16))) int hist_all[SF_WAVES][SEL_WHIST];
  // rows of a batch are handed out one at a time (a counter per batch
  // parity), so a wave with cheap rows takes more of them
  __shared__ int sNext[2];
  __shared__ int sSz[SEL_NC];  // the head's key-cluster sizes

  const int h = blockIdx.y;
  const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int jl = l & 31, hh = l >> 5;
  int* hist = hist_all[wv];
  const int32_t* offh = off + (size_t)h * (CQ + 1);
  int lim = offh[CQ];
  if (lim > N) lim = N;  // qcounts summing past N is invalid input; never read past N
  const int base = blockIdx.x * SF_ROWS * SF_BATCHES;
  if (base >= lim) return;
  // the key total
  int ktot = 0;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int32_t* p = kcounts + (size_t)h * SEL_NC + 512 * g + 8 * l;
#pragma unroll
    for (int j = 0; j < 8; ++j) ktot += p[j];
  }
  ktot = wave_sum(ktot);
  int ns = *ns_dev;
  ns = ns < 1 ? 1 : ns;
  ns = ns > ktot ? ktot : ns;
  // centroid fragments of the wave's score tiles (the A operands of
  // score_kernel: row 32 cb + jl, dims 8 hh .. and 16 + 8 hh ..): waves 0-3
  // take 6 of the 64 tiles, waves 4-11 take 5
  const int wv_u = __builtin_amdgcn_readfirstlane(wv);
  const int t0 = wv_u < 4 ? 6 * wv_u : 24 + 5 * (wv_u - 4);
  const int ntl = wv_u < 4 ? 6 : 5;
  const uint16_t* ch = cks + ((size_t)h * SEL_NC + 32 * t0 + jl) * 32 + 8 * hh;
  const int32_t* qp = qperm + (size_t)h * N;
  const uint16_t* qh = QU + (size_t)h * N * 32;
  int32_t* uh = unip + (size_t)h * CQ * (SEL_NC / 32);
  int t = -1, tend = 0;
  uint32_t acc = 0;
  int klo = SEL_NO_BOUND, vstar = 0;  // lower-bound guess from the previous row
  // projected query rows of a batch (the B operands): lane jl's row, dims
  // 8 hh .. and 16 + 8 hh ..
  auto load_rows = [&](int j0, u32x4& b0, u32x4& b1) {
    const int row = j0 + jl;
    b0 = u32x4{0u, 0u, 0u, 0u};
    b1 = u32x4{0u, 0u, 0u, 0u};
    if (row < lim) {
      const uint16_t* qr = qh + (size_t)qp[row] * 32 + 8 * hh;
      b0 = *(const u32x4*)(qr);
      b1 = *(const u32x4*)(qr + 16);
    }
  };
  u32x4 b0, b1;
  load_rows(base, b0, b1);
  auto load_ca = [&](u32x4 (&ca0)[SF_TILES], u32x4 (&ca1)[SF_TILES]) {
#pragma unroll
    for (int cb = 0; cb < SF_TILES; ++cb) {
      ca0[cb] = ca1[cb] = u32x4{0u, 0u, 0u, 0u};
      if (cb < ntl) {
        ca0[cb] = *(const u32x4*)(ch + cb * 32 * 32);
        ca1[cb] = *(const u32x4*)(ch + cb * 32 * 32 + 16);
      }
    }
  };

  // the wave's centroid fragments of the next batch, loaded while the wave
  // waits at the end of the previous batch (its selection registers are dead
  // there), so their L2 latency hides behind that barrier
  u32x4 ca0[SF_TILES], ca1[SF_TILES];
  load_ca(ca0, ca1);
  if (threadIdx.x < 2) sNext[threadIdx.x] = 0;
  for (int c = threadIdx.x; c < SEL_NC; c += SF_WAVES * 64) sSz[c] = kcounts[(size_t)h * SEL_NC + c];
  for (int b = 0; b < SF_BATCHES; ++b) {
    const int j0 = base + SF_ROWS * b;
    if (j0 >= lim) break;
    {  // scores of rows j0 .. j0 + 31 against the wave's centroids -> keys in LDS
      uint16_t* krow = sKey + jl * SF_PITCH + 4 * hh;
#pragma unroll
      for (int cb = 0; cb < SF_TILES; ++cb) {
        if (cb >= ntl) break;  // wave-uniform
        f32x16 sc = zero16();
        sc = Mfma<F16T>::run(ca0[cb], b0, sc);
        sc = Mfma<F16T>::run(ca1[cb], b1, sc);
        // lane holds centroids 32 cb + 8 g + 4 hh + e (e < 4) of row jl
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x2 o;
          o[0] = Pk<F16T>::pack(sc[4 * g + 0], sc[4 * g + 1]);  // fp32 -> fp16, RNE
          o[1] = Pk<F16T>::pack(sc[4 * g + 2], sc[4 * g + 3]);
#pragma unroll
          for (int w = 0; w < 2; ++w) o[w] = key_pair(o[w]);  // ordered keys of both halves
          *(u32x2*)(krow + key_col(32 * (t0 + cb) + 8 * g, jl & 15)) = o;
        }
      }
    }
    // the next batch's rows load while this batch is selected
    load_rows(j0 + SF_ROWS, b0, b1);
    __syncthreads();
    // every wave is past the previous batch: its counter can be reset
    if (threadIdx.x == 0) sNext[(b + 1) & 1] = 0;
    // the next row is taken from the counter while the current one is
    // selected, so the atomic's latency is hidden
    auto grab = [&]() {
      int r = 0;
      if (l == 0) r = atomicAdd(&sNext[b & 1], 1);
      return r;
    };
    int rnext = grab();
#pragma unroll 1
    for (;;) {
      const int r = __builtin_amdgcn_readfirstlane(rnext);
      const int j = j0 + r;
      if (r >= SF_ROWS || j >= lim) break;  // wave-uniform (rows only grow per wave)
      rnext = grab();
      if (j >= tend) {      // wave-uniform: every lane takes part in the shuffles
        if (t >= 0) flush_union(acc, uh + (size_t)t * (SEL_NC / 32));
        acc = 0;
        if (t < 0) {  // query cluster of the first row: largest t with off[t] <= j
          int lo = 0, hi = CQ - 1;
          while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (offh[mid] <= j) lo = mid; else hi = mid - 1;
          }
          t = lo;
        }
        while (t < CQ - 1 && offh[t + 1] <= j) ++t;  // next non-empty cluster
        tend = offh[t + 1];
      }
      uint32_t kp[16];
      const uint16_t* kr = sKey + r * SF_PITCH;
      const int rsw = r & 15;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x4 v = *(const u32x4*)(kr + key_col(512 * g + 8 * l, rsw));
#pragma unroll
        for (int q = 0; q < 4; ++q) kp[4 * g + q] = v[q];
      }
      int rc;
      // the window around the previous row's crossing first; the full search
      // when the crossing lies outside it (or for the wave's first row)
      int vs, wgt, weq, ntie;
      int where = 0, bits_ok = 0;
      uint32_t bits = 0;
      if (klo != SEL_NO_BOUND) {
        const int lo = vstar - SEL_WIN / 2;
        where = window_cross(kp, kr, rsw, sSz, hist, ns, lo, &vs, &wgt, &weq, &ntie, &bits, &bits_ok);
        if (where > 0)  // the crossing is above the window: the window above it
          where = window_cross(kp, kr, rsw, sSz, hist, ns, lo + SEL_WIN, &vs, &wgt, &weq, &ntie, &bits,
                               &bits_ok);
        else if (where < 0)  // below it: the window below
          where = window_cross(kp, kr, rsw, sSz, hist, ns, lo - SEL_WIN, &vs, &wgt, &weq, &ntie, &bits,
                               &bits_ok);
      }
      if (where != 0 || klo == SEL_NO_BOUND) {
        radix_cross(kp, sSz, hist, ns, klo, &vs, &wgt, &weq, &ntie);
        bits_ok = 0;
      }
      vstar = vs;
      if (bits_ok) {  // wave-uniform
        rc = wgt + weq;
        acc |= bits;
      } else {
        acc |= select_bits(kp, sSz, ns, vstar, wgt, weq, ntie, &rc);
      }
      klo = vstar - SEL_BOUND_MARGIN;
      if (l == 0) rowcnt[(size_t)h * N + qp[j]] = rc;
    }
    load_ca(ca0, ca1);  // the next batch's fragments (see above)
    __syncthreads();  // the next batch overwrites the keys
  }
  if (t >= 0) flush_union(acc, uh + (size_t)t * (SEL_NC / 32));
}

__global__ void expand_union_kernel(const int32_t* __restrict__ unip, uint8_t* __restrict__ uni,
                                    long long nbits) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < nbits;
       i += (long long)gridDim.x * blockDim.x)
    uni[i] = (uint8_t)(((uint32_t)unip[i >> 5] >> (i & 31)) & 1u);
}

extern "C" size_t t2t_select_ws_bytes(int H, int N, int CQ) {
  (void)N;
  WsCarver w(nullptr);
  w.take<int32_t>((size_t)H * (CQ + 1));          // query-cluster offsets
  w.take<int32_t>((size_t)H * CQ * (SEL_NC / 32)); // packed union for t2t_select_run
  return w.off;
}

static int select_common(const void* gl, const int32_t* kcounts, const int32_t* qperm,
                         const int32_t* qcounts, const int32_t* ns_dev, int32_t* unip,
                         int32_t* rowcnt, int H, int N, int CQ, void* ws, size_t ws_bytes,
                         hipStream_t st) {
  T2T_REQUIRE(gl && kcounts && qperm && qcounts && ns_dev && unip && rowcnt,
              "select: null pointer");
  T2T_REQUIRE(H > 0 && N > 0 && CQ > 0, "select: H=%d N=%d CQ=%d", H, N, CQ);
  T2T_REQUIRE(N < 524288, "select: N=%d must be < 524288", N);
  if (!ws || ws_bytes < t2t_select_ws_bytes(H, N, CQ)) {
    t2t_set_error("select: workspace %zu < %zu bytes", ws_bytes, t2t_select_ws_bytes(H, N, CQ));
    return T2T_ERR_WORKSPACE;
  }
  WsCarver w(ws);
  int32_t* off = w.take<int32_t>((size_t)H * (CQ + 1));
  hipLaunchKernelGGL(select_prep_kernel, dim3(H), dim3(1024), 0, st, qcounts, off, unip, CQ);
  T2T_LAUNCH_CHECK("select_prep");
  const int rows_per_block = SEL_WAVES * SEL_ROWS_PER_WAVE;
  hipLaunchKernelGGL(select_main_kernel, dim3(cdiv(N, rows_per_block), H), dim3(SEL_WAVES * 64), 0,
                     st, (const uint16_t*)gl, kcounts, qperm, off, ns_dev, unip, rowcnt, N, CQ);
  T2T_LAUNCH_CHECK("select_main");
  return T2T_OK;
}

static int score_select_launch(const void* QU, const void* cks, const int32_t* kcounts,
                               const int32_t* qperm, const int32_t* qcounts,
                               const int32_t* ns_dev, int32_t* unip, int32_t* rowcnt, int H,
                               int N, int CQ, int32_t* off, hipStream_t st) {
  hipLaunchKernelGGL(select_prep_kernel, dim3(H), dim3(1024), 0, st, qcounts, off, unip, CQ);
  T2T_LAUNCH_CHECK("score_select prep");
  hipLaunchKernelGGL(score_select_kernel, dim3(cdiv(N, SF_ROWS * SF_BATCHES), H),
                     dim3(SF_WAVES * 64), 0, st, (const uint16_t*)QU, (const uint16_t*)cks,
                     kcounts, qperm, off, ns_dev, unip, rowcnt, N, CQ);
  T2T_LAUNCH_CHECK("score_select");
  return T2T_OK;
}

extern "C" int t2t_score_select_packed(const void* QU, const void* cks, const int32_t* kcounts,
                                       const int32_t* qperm, const int32_t* qcounts,
                                       const int32_t* ns_dev, int32_t* unip, int32_t* rowcnt,
                                       int H, int N, int CQ, void* ws, size_t ws_bytes,
                                       void* stream) {
  T2T_REQUIRE(QU && cks && kcounts && qperm && qcounts && ns_dev && unip && rowcnt,
              "score_select: null pointer");
  T2T_REQUIRE(H > 0 && N > 0 && CQ > 0, "score_select: H=%d N=%d CQ=%d", H, N, CQ);
  T2T_REQUIRE(N < 524288, "score_select: N=%d must be < 524288", N);
  if (!ws || ws_bytes < t2t_select_ws_bytes(H, N, CQ)) {
    t2t_set_error("score_select: workspace %zu < %zu bytes", ws_bytes,
                  t2t_select_ws_bytes(H, N, CQ));
    return T2T_ERR_WORKSPACE;
  }
  WsCarver w(ws);
  int32_t* off = w.take<int32_t>((size_t)H * (CQ + 1));
  return score_select_launch(QU, cks, kcounts, qperm, qcounts, ns_dev, unip, rowcnt, H, N, CQ, off,
                             (hipStream_t)stream);
}

// ---- the allocation-free variant -------------------------------------------
// Its only scratch (the query-cluster offsets, H * (CQ + 1) int32) lives in a
// file-scope device array.  Every GPU holds its own copy of the array at its
// own address; the host keeps that address per device, taken once with
// hipGetSymbolAddress while the device is current (the array's name is not a
// device address in host code).  select_prep_kernel writes every offset of
// the call before the selection reads it, so nothing needs clearing.  Calls
// that overlap on one GPU share the array and race.
static __device__ __align__(256) int32_t scratch[T2T_NOALLOC_SCRATCH_INTS];

#define T2T_MAX_DEVICES 64
static std::mutex g_scratch_mu;
static int32_t* g_scratch_ptr[T2T_MAX_DEVICES];

static int noalloc_scratch(hipStream_t stream, int32_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    t2t_set_error("score_select_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return T2T_ERR_LAUNCH;
  }
  // The scratch address is per device: a stream of another GPU would receive
  // a pointer into this GPU's copy of the array.
  hipDevice_t sdev = -1;
  e = hipStreamGetDevice(stream, &sdev);
  if (e != hipSuccess) {
    t2t_set_error("score_select_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
    return T2T_ERR_LAUNCH;
  }
  if ((int)sdev != dev) {
    t2t_set_error("score_select_noalloc: stream belongs to device %d, current device is %d",
                  (int)sdev, dev);
    return T2T_ERR_UNSUPPORTED;
  }
  if (dev < 0 || dev >= T2T_MAX_DEVICES) {
    t2t_set_error("score_select_noalloc: device %d outside [0, %d)", dev, T2T_MAX_DEVICES);
    return T2T_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      t2t_set_error("score_select_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return T2T_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = (int32_t*)p;
  }
  *out = g_scratch_ptr[dev];
  return T2T_OK;
}

extern "C" size_t t2t_score_select_noalloc_max_ints(void) { return T2T_NOALLOC_SCRATCH_INTS; }

extern "C" int t2t_score_select_packed_noalloc(const void* QU, const void* cks,
                                               const int32_t* kcounts, const int32_t* qperm,
                                               const int32_t* qcounts, const int32_t* ns_dev,
                                               int32_t* unip, int32_t* rowcnt, int H, int N,
                                               int CQ, void* stream) {
  T2T_REQUIRE(QU && cks && kcounts && qperm && qcounts && ns_dev && unip && rowcnt,
              "score_select_noalloc: null pointer");
  T2T_REQUIRE(H > 0 && N > 0 && CQ > 0, "score_select_noalloc: H=%d N=%d CQ=%d", H, N, CQ);
  T2T_REQUIRE(N < 524288, "score_select_noalloc: N=%d must be < 524288", N);
  if ((size_t)H * (size_t)(CQ + 1) > (size_t)T2T_NOALLOC_SCRATCH_INTS) {
    t2t_set_error("score_select_noalloc: H * (CQ + 1) = %zu offsets exceed the %d-entry "
                  "static scratch (use t2t_score_select_packed with a workspace)",
                  (size_t)H * (size_t)(CQ + 1), T2T_NOALLOC_SCRATCH_INTS);
    return T2T_ERR_UNSUPPORTED;
  }
  int32_t* off = nullptr;
  int rc = noalloc_scratch((hipStream_t)stream, &off);
  if (rc) return rc;
  return score_select_launch(QU, cks, kcounts, qperm, qcounts, ns_dev, unip, rowcnt, H, N, CQ, off,
                             (hipStream_t)stream);
}

extern "C" int t2t_select_run_packed(const void* gl, const int32_t* kcounts, const int32_t* qperm,
                                     const int32_t* qcounts, const int32_t* ns_dev, int32_t* unip,
                                     int32_t* rowcnt, int H, int N, int CQ, void* ws,
                                     size_t ws_bytes, void* stream) {
  return select_common(gl, kcounts, qperm, qcounts, ns_dev, unip, rowcnt, H, N, CQ, ws, ws_bytes,
                       (hipStream_t)stream);
}

extern "C" int t2t_select_run_split_packed(const void* gl, const int32_t* kcounts,
                                           const int32_t* qperm, const int32_t* qcounts, int cap,
                                           const int32_t* ns_dev, int32_t* unip, int32_t* rowcnt,
                                           int H, int N, int CQ, void* ws, size_t ws_bytes,
                                           void* stream) {
  T2T_REQUIRE(cap >= 1, "select split: cap=%d must be >= 1", cap);
  return select_common(gl, kcounts, qperm, qcounts, ns_dev, unip, rowcnt, H, N, CQ, ws, ws_bytes,
                       (hipStream_t)stream);
}

extern "C" int t2t_select_run(const void* gl, const int32_t* kcounts, const int32_t* qperm,
                              const int32_t* qcounts, const int32_t* ns_dev, uint8_t* uni,
                              int32_t* rowcnt, int H, int N, int CQ, void* ws, size_t ws_bytes,
                              void* stream) {
  T2T_REQUIRE(uni, "select run: null uni");
  if (!ws || ws_bytes < t2t_select_ws_bytes(H, N, CQ)) {
    t2t_set_error("select run: workspace %zu < %zu bytes", ws_bytes, t2t_select_ws_bytes(H, N, CQ));
    return T2T_ERR_WORKSPACE;
  }
  WsCarver w(ws);
  w.take<int32_t>((size_t)H * (CQ + 1));
  int32_t* packed = w.take<int32_t>((size_t)H * CQ * (SEL_NC / 32));
  int rc = select_common(gl, kcounts, qperm, qcounts, ns_dev, packed, rowcnt, H, N, CQ, ws,
                         ws_bytes, (hipStream_t)stream);
  if (rc) return rc;
  const long long nbits = (long long)H * CQ * SEL_NC;
  hipLaunchKernelGGL(expand_union_kernel, dim3(2048), dim3(256), 0, (hipStream_t)stream, packed,
                     uni, nbits);
  T2T_LAUNCH_CHECK("select run expand");
  return T2T_OK;
}
