// Shared device/host helpers for the femtohip kernels (gfx950, wave64).
//
// Element types: bf16 is carried as raw uint16_t bits (round-to-nearest-even
// conversion, the same rounding torch applies when it narrows fp32 results to
// bfloat16), fp32 as float.  Every kernel computes in fp32 registers and rounds
// only where the Hugging Face Llama layer (transformers 5.15.0,
// models/llama/modeling_llama.py) materialises a bf16 tensor.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "femtohip.h"

namespace fh {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 bits
__device__ __forceinline__ float bf2f(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16 (NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// Two floats rounded to bf16 and packed (a in the low half) by one
// v_cvt_pk_bf16_f32; same rounding as f2bf.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// ------------------------------------------------------ fast division
// n / d for 32-bit n by a runtime divisor fixed per launch: with
// M = ceil(2^64 / d), n / d = floor(M * n / 2^64) exactly for every 32-bit n
// and 1 < d < 2^32 (Lemire, Kaser, Kurz, "Faster Remainder by Direct
// Computation", 2019).  M is computed on the host; d == 1 is special-cased.
struct FastDiv {
  uint64_t m;
  uint32_t d;
  FastDiv() = default;
  __host__ explicit FastDiv(uint32_t div) : m(div > 1 ? ~uint64_t(0) / div + 1 : 0), d(div) {}
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    return d == 1 ? n : static_cast<uint32_t>(__umul64hi(m, n));
  }
};

// ------------------------------------------------------- element traits
// Elem<T>::load8 / store8 move 8 consecutive elements between memory and
// fp32 registers with 128-bit accesses (one dwordx4 for bf16, two for fp32).
template <typename T>
struct Elem;

template <>
struct Elem<uint16_t> {
  static constexpr fh_dtype kDtype = FH_BF16;
  // 8 elements as loaded (kept packed in registers until needed).
  using Raw = uint4;
  __device__ __forceinline__ static Raw ldraw(const uint16_t* p) {
    return *reinterpret_cast<const uint4*>(p);
  }
  // ldraw as a non-temporal (streaming) load: data read once.
  __device__ __forceinline__ static Raw ldraw_stream(const uint16_t* p) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
  }
  __device__ __forceinline__ static void unpack(const Raw& q, float v[8]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void load8(const uint16_t* p, float v[8]) {
    const uint4 q = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  // 8 floats rounded to bf16 and packed (exact for bf16-representable values).
  __device__ __forceinline__ static Raw pack(const float v[8]) {
    return make_uint4(pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3]), pk_bf16(v[4], v[5]),
                      pk_bf16(v[6], v[7]));
  }
  __device__ __forceinline__ static void straw(uint16_t* p, const Raw& q) {
    *reinterpret_cast<uint4*>(p) = q;
  }
  __device__ __forceinline__ static void store8(uint16_t* p, const float v[8]) {
    straw(p, pack(v));
  }
  // Rounds a value to the precision a tensor of this dtype would hold.
  __device__ __forceinline__ static float rnd(float f) { return round_bf(f); }
  __device__ __forceinline__ static float ld1(const uint16_t* p) { return bf2f(*p); }
  __device__ __forceinline__ static void st1(uint16_t* p, float f) { *p = f2bf(f); }
};

template <>
struct Elem<float> {
  static constexpr fh_dtype kDtype = FH_F32;
  struct Raw {
    float4 a, b;
  };
  __device__ __forceinline__ static Raw ldraw(const float* p) {
    return Raw{*reinterpret_cast<const float4*>(p), *reinterpret_cast<const float4*>(p + 4)};
  }
  __device__ __forceinline__ static Raw ldraw_stream(const float* p) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    const v4f a = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p));
    const v4f b = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p + 4));
    return Raw{make_float4(a.x, a.y, a.z, a.w), make_float4(b.x, b.y, b.z, b.w)};
  }
  __device__ __forceinline__ static void unpack(const Raw& q, float v[8]) {
    v[0] = q.a.x; v[1] = q.a.y; v[2] = q.a.z; v[3] = q.a.w;
    v[4] = q.b.x; v[5] = q.b.y; v[6] = q.b.z; v[7] = q.b.w;
  }
  __device__ __forceinline__ static void load8(const float* p, float v[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  __device__ __forceinline__ static Raw pack(const float v[8]) {
    return Raw{make_float4(v[0], v[1], v[2], v[3]), make_float4(v[4], v[5], v[6], v[7])};
  }
  __device__ __forceinline__ static void straw(float* p, const Raw& q) {
    *reinterpret_cast<float4*>(p) = q.a;
    *reinterpret_cast<float4*>(p + 4) = q.b;
  }
  __device__ __forceinline__ static void store8(float* p, const float v[8]) {
    straw(p, pack(v));
  }
  __device__ __forceinline__ static float rnd(float f) { return f; }
  __device__ __forceinline__ static float ld1(const float* p) { return *p; }
  __device__ __forceinline__ static void st1(float* p, float f) { *p = f; }
};

// ------------------------------------------------------------ RoPE pair
// Rotate-half rotary embedding of one pair (x0 at dim i, x1 at dim
// i + head_dim/2; cos c0, c1 and sin s0, s1 at those dims), rounded with
// Elem<T>::rnd wherever the reference materialises a tensor -- each product,
// then the sum (q*cos + rotate_half(q)*sin, modeling_llama.py:130-160):
//   forward:   o0 = x0*c0 - x1*s0,  o1 = x1*c1 + x0*s1
//   backward (the transposed rotation, grad*cos + rotate_half^T(grad*sin)):
//              o0 = x0*c0 + x1*s1,  o1 = x1*c1 - x0*s0
// Multiply-add contraction is off, so the fp32 path also rounds each product
// separately, as torch's elementwise ops do.
template <typename T, bool BWD>
__device__ __forceinline__ void rope_pair(float x0, float x1, float c0, float c1, float s0, float s1,
                                          float& o0, float& o1) {
#pragma clang fp contract(off)
  using E = Elem<T>;
  if constexpr (!BWD) {
    o0 = E::rnd(E::rnd(x0 * c0) - E::rnd(x1 * s0));
    o1 = E::rnd(E::rnd(x1 * c1) + E::rnd(x0 * s1));
  } else {
    o0 = E::rnd(E::rnd(x0 * c0) + E::rnd(x1 * s1));
    o1 = E::rnd(E::rnd(x1 * c1) - E::rnd(x0 * s0));
  }
}

// One output of the forward rotation for a caller that holds its own element
// x, the pair partner p, and cos c / sin s at its own dim: the lower half's
// o0 = x*c - p*s and the upper half's o1 = x*c + p*s, rounded as rope_pair
// rounds.  Round-to-nearest-even is symmetric, so rnd(p*s) negated equals
// rnd(p*(-s)) and the caller passes s_signed = -s (lower) or s (upper): one
// form covers both halves bit for bit.
template <typename T>
__device__ __forceinline__ float rope_fwd_one(float x, float p, float c, float s_signed) {
#pragma clang fp contract(off)
  using E = Elem<T>;
  return E::rnd(E::rnd(x * c) + E::rnd(p * s_signed));
}

// ------------------------------------------------------- wave reductions
// DPP (data-parallel primitive) lane moves: VALU ops with no LDS round trip.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes of a wave, returned to every lane: quad swaps, half-row
// and row mirrors give each 16-lane row its sum, row_bcast15/31 carry rows into
// lane 63, and readlane broadcasts it.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);         // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);         // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);        // row_half_mirror
  v += dpp<0x140>(v);        // row_mirror
  v += dpp<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
  v += dpp<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// ------------------------------------------------------- host-side status
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

}  // namespace fh

#define FH_REQUIRE(cond, msg)                                   \
  do {                                                          \
    if (!(cond)) return ::fh::fail(FH_ERR_INVALID, (msg));      \
  } while (0)
