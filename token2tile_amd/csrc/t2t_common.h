// Shared device helpers for the gfx950 Token2Tile kernels: element types,
// MFMA wrappers, wave64 reductions and host-side error plumbing.
#pragma once
#include <hip/hip_runtime.h>
#include <climits>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>
#include <stddef.h>
#include "../../include/t2t_hip.h"

#define T2T_WAVE 64

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// element types: raw 16-bit storage, conversions through fp32
// ---------------------------------------------------------------------------
struct F16T {
  static constexpr int code = T2T_F16;
  __device__ static inline float to_f(uint16_t u) {
    _Float16 h = __builtin_bit_cast(_Float16, u);
    return (float)h;
  }
  __device__ static inline uint16_t from_f(float f) {  // round to nearest even
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
  }
};
struct BF16T {
  static constexpr int code = T2T_BF16;
  __device__ static inline float to_f(uint16_t u) {
    return __builtin_bit_cast(float, (uint32_t)u << 16);
  }
  __device__ static inline uint16_t from_f(float f) {  // round to nearest even (v_cvt_pk_bf16_f32)
    return __builtin_bit_cast(uint16_t, (__bf16)f);
  }
};

__device__ inline float h2f(uint16_t u) { return F16T::to_f(u); }

// Materialise an fp32 value: keeps the compiler from fusing the operation
// that produced it with a following fp16 conversion into one mixed-precision
// instruction (which rounds once instead of fp32-then-fp16).
__device__ inline float opaque(float x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ inline uint16_t f2h(float f) { return F16T::from_f(f); }

// bf16 -> fp16 (through fp32; exact for values inside the fp16 normal range)
__device__ inline uint16_t bf2h(uint16_t b) { return f2h(BF16T::to_f(b)); }

// ---------------------------------------------------------------------------
// MFMA 32x32x16 (gfx950).  Operand convention used everywhere:
//   lane l supplies A[i = l % 32][k = 8 * (l / 32) + t] and
//   B[k = 8 * (l / 32) + t][j = l % 32] for t = 0..7;
//   D[i][j] lands in lane l = j + 32 * ((i / 4) % 2), element
//   a = 4 * (i / 8) + i % 4  (i = 8 * (a / 4) + 4 * (l / 32) + a % 4).
// ---------------------------------------------------------------------------
template <typename T> struct Mfma;
template <> struct Mfma<F16T> {
  __device__ static inline f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma<BF16T> {
  __device__ static inline f32x16 run(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

// Two floats -> one packed pair of T (round to nearest even, one
// v_cvt_pk_* instruction), and the sum of a packed pair added to acc (dot2
// with (1, 1), fp32 accumulation).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <typename T> struct Pk;
template <> struct Pk<F16T> {
  __device__ static inline uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  }
  __device__ static inline float sum2(uint32_t p, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, p), (f16x2){(_Float16)1.0f, (_Float16)1.0f},
                                  acc, false);
  }
};
template <> struct Pk<BF16T> {
  __device__ static inline uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  }
  __device__ static inline float sum2(uint32_t p, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p),
                                           (bf16x2){(__bf16)1.0f, (__bf16)1.0f}, acc, false);
  }
};

__device__ inline f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// ---------------------------------------------------------------------------
// wave64 helpers
// ---------------------------------------------------------------------------
__device__ inline int lane_id() { return __lane_id(); }

// Cross-lane steps run on DPP (data-parallel primitives: a VALU operand read
// from another lane of the same row of 16, or a row broadcast), not through
// LDS permutes.  Every helper below must be called by the whole wave.
//   row_shr:n  0x110 + n   lane i of each row reads lane i - n of that row
//                          (lanes i < n read the identity)
//   row_bcast:15  0x142    rows 1..3 read lane 15 of the previous row
//   row_bcast:31  0x143    rows 2, 3 read lane 31
// An inclusive scan is the four in-row shifts and the two broadcasts (rows 1
// and 3 take row 0's and row 2's total, then rows 2 and 3 take lanes 0..31's).
template <typename F>
__device__ inline int wave_incl_scan_op(int x, int ident, F op) {
  x = op(x, __builtin_amdgcn_update_dpp(ident, x, 0x111, 0xf, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(ident, x, 0x112, 0xf, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(ident, x, 0x114, 0xf, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(ident, x, 0x118, 0xf, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(ident, x, 0x142, 0xa, 0xf, false));
  x = op(x, __builtin_amdgcn_update_dpp(ident, x, 0x143, 0xc, 0xf, false));
  return x;
}
__device__ inline int wave_incl_scan(int v) {
  return wave_incl_scan_op(v, 0, [](int a, int b) { return a + b; });
}
__device__ inline int wave_incl_max(int v) {
  return wave_incl_scan_op(v, INT_MIN, [](int a, int b) { return a > b ? a : b; });
}
// total over the wave, the same (scalar) value in every lane
__device__ inline int wave_sum(int v) { return __builtin_amdgcn_readlane(wave_incl_scan(v), 63); }
// v_permlane32_swap_b32 with both operands v leaves {v[l], v[l ^ 32]} in every
// lane l (in an order that depends on the half), so symmetric combinations of a
// lane and its partner in the other half take one exchange
__device__ inline float half_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                                 __builtin_bit_cast(uint32_t, v), false, false);
  return __builtin_elementwise_maximum(__builtin_bit_cast(float, (uint32_t)r[0]),
                                       __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ inline float half_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                                 __builtin_bit_cast(uint32_t, v), false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}
// the value of lane l ^ 32
__device__ inline uint32_t half_partner(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __lane_id() < 32 ? (uint32_t)r[1] : (uint32_t)r[0];
}
__device__ inline long long wave_sum64(long long v) {
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
  return v;
}

// fp16 score -> int16 key ordering like the value with -0 < +0
__device__ inline int score_key(uint16_t u) {
  u ^= (uint16_t)(((u >> 15) & 1u) * 0x7FFFu);
  return (int)(int16_t)u;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
void t2t_set_error(const char* fmt, ...);
int t2t_check_launch(const char* what);

#define T2T_REQUIRE(cond, ...)              \
  do {                                      \
    if (!(cond)) {                          \
      t2t_set_error(__VA_ARGS__);           \
      return T2T_ERR_ARG;                   \
    }                                       \
  } while (0)

#define T2T_LAUNCH_CHECK(what)                          \
  do {                                                  \
    int _rc = t2t_check_launch(what);                   \
    if (_rc != T2T_OK) return _rc;                      \
  } while (0)

static inline size_t t2t_align256(size_t x) { return (x + 255) & ~(size_t)255; }
static inline int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

// Carves aligned sub-buffers out of a caller-owned workspace (base may be
// NULL to measure the size).
struct WsCarver {
  char* base;
  size_t off = 0;
  explicit WsCarver(void* b) : base((char*)b) {}
  template <typename T> T* take(size_t count) {
    T* p = base ? (T*)(base + off) : nullptr;
    off += t2t_align256(count * sizeof(T));
    return p;
  }
};
