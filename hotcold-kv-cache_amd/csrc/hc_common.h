// Shared device/host helpers for the gfx950 hot-tier kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>
#include <utility>

#include "hotcold_hip.h"

namespace hc {

typedef _Float16 half_t;
typedef __bf16 bf16_t;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Host-side error reporting (defined in hc_runtime.hip).
// ---------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);
int dtype_size(int dtype);

#define HC_REQUIRE(cond, ...)                                        \
  do {                                                               \
    if (!(cond)) return ::hc::set_error(HC_ERR_INVALID, __VA_ARGS__); \
  } while (0)

// ---------------------------------------------------------------------------
// Element conversions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(half_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ half_t from_f32<half_t>(float x) { return (half_t)x; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return (bf16_t)x; }

__device__ __forceinline__ double to_f64(float x) { return (double)x; }
__device__ __forceinline__ double to_f64(half_t x) { return (double)(float)x; }
__device__ __forceinline__ double to_f64(bf16_t x) { return (double)(float)x; }

// ---------------------------------------------------------------------------
// Vectorised 16-byte loads/stores (global_load_dwordx4).
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// Unpack n contiguous elements of T from raw 32-bit words into floats.
template <typename T>
struct Unpack;
template <>
struct Unpack<half_t> {
  __device__ __forceinline__ static float get(const uint32_t* w, int i) {
    uint32_t word = w[i >> 1];
    uint16_t bits = (i & 1) ? (uint16_t)(word >> 16) : (uint16_t)(word & 0xffffu);
    return (float)__builtin_bit_cast(half_t, bits);
  }
};
template <>
struct Unpack<bf16_t> {
  __device__ __forceinline__ static float get(const uint32_t* w, int i) {
    uint32_t word = w[i >> 1];
    uint32_t bits = (i & 1) ? (word & 0xffff0000u) : (word << 16);
    return __builtin_bit_cast(float, bits);
  }
};
template <>
struct Unpack<float> {
  // __uint_as_float takes the word by value: __builtin_bit_cast of an
  // element of a register-resident array miscompiles with this toolchain
  // (it reads element 0).
  __device__ __forceinline__ static float get(const uint32_t* w, int i) { return __uint_as_float(w[i]); }
};

// ---------------------------------------------------------------------------
// Wave64 reductions (ds_swizzle / bpermute through __shfl_xor).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    lo = __shfl_xor(lo, o, 64);
    hi = __shfl_xor(hi, o, 64);
    v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

// ---------------------------------------------------------------------------
// Deterministic exp for x <= 0 (the softmax numerators of the window scores).
//
// Cody-Waite argument reduction x = k*ln2 + r with the two-part ln2 split of
// fdlibm (ln2_hi has 32 significant bits so k*ln2_hi is exact for |k| < 2^21),
// then the degree-12 Taylor polynomial of exp(r) on |r| <= ln2/2 in Horner
// form, then the exact scaling by 2^k.  Every step is an IEEE-754 binary64
// fma/mul/add with round-to-nearest-even, so any conforming implementation
// (this kernel, the C restatement used for testing) produces identical bits.
// Inputs below -708 return 0 (their fixed-point contribution is 0 anyway).
// ---------------------------------------------------------------------------
#define HC_LN2_HI 6.93147180369123816490e-01
#define HC_LN2_LO 1.90821492927058770002e-10
#define HC_INV_LN2 1.44269504088896338700e+00

// The constants (ln2 split, 1/ln2, the 13 Taylor coefficients 1/12! .. 1/0!
// highest degree first) are read once per kernel from constant memory into
// SGPRs (DetExp::load), so each Horner step is one v_fma_f64 with an SGPR
// operand instead of a 64-bit constant move plus v_fmac.  The out-of-range
// test is a select, not a branch: the polynomial runs on a clamped argument
// and the result is replaced by 0.
static __constant__ double kDetExpConst[18] = {
    HC_INV_LN2,
    HC_LN2_HI,
    HC_LN2_LO,
    2.08767569878680989792e-09,  // 1/12!
    2.50521083854417187751e-08,  // 1/11!
    2.75573192239858906526e-07,  // 1/10!
    2.75573192239858906526e-06,  // 1/9!
    2.48015873015873015873e-05,  // 1/8!
    1.98412698412698412698e-04,  // 1/7!
    1.38888888888888888889e-03,  // 1/6!
    8.33333333333333333333e-03,  // 1/5!
    4.16666666666666666667e-02,  // 1/4!
    1.66666666666666666667e-01,  // 1/3!
    5.00000000000000000000e-01,  // 1/2!
    1.0,                         // 1/1!
    1.0,                         // 1/0!
    17592186044416.0,            // 2^44, the fixed-point quantum's inverse
    4503599627370496.0,          // 2^52
};

struct DetExp {
  double c[18];
  __device__ static DetExp load() {
    DetExp d;
#pragma unroll
    for (int i = 0; i < 18; ++i) d.c[i] = kDetExpConst[i];
    return d;
  }
  // Polynomial part for max(x, -708): returns p in [0.7, 1.5) and k + BIAS,
  // k in [-1021, 0], with exp = p * 2^k.
  // The shifter is 1.5 * 2^52 + bias for an even bias: RNE(t + bias) =
  // RNE(t) + bias, so the low mantissa bits hold k + bias while kf is exactly
  // rint(t).
  template <int BIAS>
  __device__ __forceinline__ double poly(double x, uint32_t& kb) const {
#pragma clang fp contract(off)
    static_assert(BIAS % 2 == 0 && BIAS >= 0 && BIAS < 1024, "even exponent bias");
    constexpr double kShift = 6755399441055744.0 + BIAS;
    const double xc = __builtin_fmax(x, -708.0);  // -inf and NaN -> -708
    // rint(xc / ln2) by the 1.5 * 2^52 shifter: the sum's ulp is 1, so its
    // one rounding is round-to-nearest-even of the (separately rounded)
    // product, and the integer k sits in the low mantissa bits.
    const double t = xc * c[0];
    const double sh = t + kShift;
    const double kf = sh - kShift;
    kb = (uint32_t)__builtin_bit_cast(uint64_t, sh);
    double r = __builtin_fma(-kf, c[1], xc);
    r = __builtin_fma(-kf, c[2], r);
    double p = c[3];
#pragma unroll
    for (int i = 4; i < 16; ++i) p = __builtin_fma(p, r, c[i]);
    return p;
  }
  // p * 2^j for p in [0.7, 1.5) and j in [-1021, 44]: the result is a normal
  // double, so the scaling is exact (v_ldexp_f64, one instruction; building
  // the factor from exponent bits measured slower).
  __device__ __forceinline__ static double scale(double p, uint32_t j) { return __builtin_ldexp(p, (int)j); }
  // The contract's value: exp(x) for x >= -708, else +0.
  __device__ __forceinline__ double operator()(double x) const {
    uint32_t k;
    const double p = poly<0>(x, k);
    return x >= -708.0 ? scale(p, k) : 0.0;  // false for -inf and NaN
  }
  // The bits of rint(e * 2^44) + 2^52 for the contract's value e.  e * 2^44 = p * 2^(k+44) exactly, so one add of
  // 2^52 rounds it as fma(e, 2^44, 2^52) would.  Below -708 it uses
  // exp(-708) (~3.3e-308) instead of 0: rint(e * 2^44) is 0 for both.
  __device__ __forceinline__ uint64_t fixed_biased(double x) const {
#pragma clang fp contract(off)
    uint32_t k44;
    const double p = poly<44>(x, k44);
    return __builtin_bit_cast(uint64_t, scale(p, k44) + c[17]);
  }
};

// Fixed-point quantum of the softmax normaliser: e in [0,1] -> rint(e * 2^44).
// e * 2^44 + 2^52 lands in [2^52, 2^53) where the spacing of doubles is 1, so
// its single rounding is round-to-nearest-even of e * 2^44 and the low
// mantissa bits are that integer; HC_FIX_BIAS is the bit pattern of 2^52,
// which DetExp::fixed_biased leaves in and sums take off once.
#define HC_FIX_BIAS 0x4330000000000000ull

// Total order key for fp32 scores: larger score -> larger key; -0 == +0;
// NaN above everything (torch.topk ranks NaN highest).
__device__ __forceinline__ uint32_t order_key(float x) {
  if (x != x) return 0xffffffffu;
  if (x == 0.0f) x = 0.0f;
  const uint32_t b = __builtin_bit_cast(uint32_t, x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time
// (register arrays indexed by i stay in registers).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// ---------------------------------------------------------------------------
// Raw buffer loads.  A load whose offset is past the resource's extent returns
// zeros without a memory access, so kernels can issue every load
// unconditionally (which keeps the compiler's vmcnt waits exact) and steer
// out-of-range lanes to kOob.
// ---------------------------------------------------------------------------
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <int BYTES>
__device__ __forceinline__ void bload(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t* w) {
  if constexpr (BYTES == 16) {
    const u32x4 x = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
    w[0] = x[0]; w[1] = x[1]; w[2] = x[2]; w[3] = x[3];
  } else if constexpr (BYTES == 8) {
    const u32x2 x = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
    w[0] = x[0]; w[1] = x[1];
  } else if constexpr (BYTES == 4) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
  } else {
    w[0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
  }
}

// A 16-byte raw buffer load with a scalar (wave-uniform) offset added to the
// lane's offset.
template <int BYTES>
__device__ __forceinline__ void bload_so(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t soff, uint32_t* w) {
  static_assert(BYTES == 16, "bload_so: 16-byte loads");
  const u32x4 x = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, (int)soff, 0));
  w[0] = x[0]; w[1] = x[1]; w[2] = x[2]; w[3] = x[3];
}

// Raw buffer stores: a store whose offset is past the extent is dropped.
template <int BYTES>
__device__ __forceinline__ void bstore(__amdgpu_buffer_rsrc_t r, uint32_t off, const uint32_t* w) {
  if constexpr (BYTES == 16) {
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{w[0], w[1], w[2], w[3]}, r, (int)off, 0, 0);
  } else if constexpr (BYTES == 8) {
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{w[0], w[1]}, r, (int)off, 0, 0);
  } else if constexpr (BYTES == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(w[0], r, (int)off, 0, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16((unsigned short)w[0], r, (int)off, 0, 0);
  }
}

// Wave-aggregated LDS updates.  Radix-select keys mostly share their leading
// digits, so plain per-lane atomics on one histogram bin or one append counter
// serialise across the whole workgroup; here each wave issues one atomic for
// the lanes that agree with its first active lane.
__device__ __forceinline__ void hist_add(uint32_t* hist, uint32_t dig, bool active) {
  const uint64_t todo = __ballot(active);
  if (!todo) return;
  const int lane = __lane_id(), leader = __ffsll((unsigned long long)todo) - 1;
  const uint32_t d0 = (uint32_t)__shfl((int)dig, leader);
  const uint64_t same = __ballot(active && dig == d0);
  if (lane == leader) atomicAdd(&hist[d0], (uint32_t)__popcll(same));
  if (active && dig != d0) atomicAdd(&hist[dig], 1u);
}

// A slot of an LDS list for each lane with `want` (-1 for the others): one
// atomic per wave, lanes in lane order.
__device__ __forceinline__ int append_slot(int* counter, bool want) {
  const uint64_t m = __ballot(want);
  if (!m) return -1;
  const int lane = __lane_id(), leader = __ffsll((unsigned long long)m) - 1;
  int base = 0;
  if (lane == leader) base = atomicAdd(counter, __popcll(m));
  base = __shfl(base, leader);
  return want ? base + __popcll(m & ((1ull << lane) - 1)) : -1;
}

}  // namespace hc
