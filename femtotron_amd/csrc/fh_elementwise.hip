// Rotary embedding (in place on q and k), SwiGLU forward/backward and the
// residual add.  All three are HBM-bound streams: every thread moves 8
// elements per tensor with 128-bit loads/stores, consecutive threads touch
// consecutive 16-byte chunks, and arithmetic stays in fp32 registers with the
// reference's bf16 rounding points applied in-register.
//
// Reference arithmetic (transformers 5.15.0):
//   rotate_half / apply_rotary_pos_emb   models/llama/modeling_llama.py:130-160
//   LlamaMLP act_fn(gate)*up             models/llama/modeling_llama.py:174-176
//   SiLUActivation = F.silu              activations.py:93-103
//   residual adds                        models/llama/modeling_llama.py:317,323
#include <type_traits>

#include "fh_common.hpp"

namespace fh {
namespace {

// sigmoid(g) = 1 / (1 + 2^(-g*log2 e)) on the transcendental unit (v_exp_f32,
// v_rcp_f32, ~1 ulp each).  The accurate expf and IEEE division cost ~30 VALU
// ops per element, which made SwiGLU ALU-bound; the result is rounded to bf16
// (8-bit mantissa) where the reference rounds.  Saturates correctly: large
// negative g gives exp -> inf, rcp -> 0.
__device__ __forceinline__ float sigmoid_f(float g) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}
__device__ __forceinline__ float silu_f(float g) { return g * sigmoid_f(g); }

#ifndef FH_ROPE_HEADS_PER_THREAD
#define FH_ROPE_HEADS_PER_THREAD 1
#endif
#ifndef FH_EW_CHUNKS
#define FH_EW_CHUNKS 1
#endif
// Heads rotated per thread (RoPE) and 8-element chunks per thread (SwiGLU,
// add).  More work per thread, with all loads hoisted, measured slower at the
// TinyLlama shapes (RoPE 4.95 -> 4.60 TB/s at 4 heads, SwiGLU fwd 5.46 -> 4.98
// at 2 chunks): more, shorter waves hide HBM latency better here.
constexpr int kRopeHG = FH_ROPE_HEADS_PER_THREAD;
constexpr int kChunks = FH_EW_CHUNKS;

// Flat chunk index -> (row, first column) of a row-strided [rows, cols]
// operand.  Index spaces below 2^32 (every layer shape) use the host-computed
// multiplier; WIDE launches keep 64-bit division.
template <bool WIDE>
__device__ __forceinline__ void row_col(int64_t idx, int cpr, const FastDiv& fd, int64_t& r,
                                        int& c) {
  if constexpr (WIDE) {
    r = idx / cpr;
    c = static_cast<int>(idx - r * cpr) * 8;
  } else {
    const uint32_t i = static_cast<uint32_t>(idx), q = fd.div(i);
    r = q;
    c = static_cast<int>(i - q * static_cast<uint32_t>(cpr)) * 8;
  }
}

// SwiGLU's inputs are read once: non-temporal loads.  Kernel-only, warm
// step shapes (T = 16384, F = 5632): forward 95.6 -> 82.6 us, backward 200 ->
// 197 us; cold at config 2: forward 54.5 -> 55.0, backward 110 -> 102 us.  The
// same loads in the add and RMSNorm kernels measured no different.
template <typename T>
__device__ __forceinline__ typename Elem<T>::Raw sw_load(const T* p) {
  return Elem<T>::ldraw_stream(p);
}

inline bool wide(int64_t n) { return n >= (int64_t(1) << 32); }

// One thread = 8 rotation pairs (i, i + d/2) of up to kRopeHG heads of one
// token: cos/sin for the pairs are loaded once and reused across the heads,
// and all the heads' loads are issued before the first store.
// Index maps of one launch: token = idx / per_tok, head group = rem / cpp,
// position = token % seq_len (host-computed multipliers; WIDE launches, whose
// index space exceeds 32 bits, divide in 64 bits).
struct RopeDivs {
  FastDiv per_tok, cpp, seq;
};

template <typename T, bool BWD, bool WIDE>
__global__ __launch_bounds__(256) void k_rope(T* __restrict__ qk, int64_t ld, int64_t tokens,
                                              int64_t seq_len, int n_heads, int head_dim,
                                              const T* __restrict__ cosv,
                                              const T* __restrict__ sinv, int cos_per_token,
                                              RopeDivs dv) {
  const int cpp = head_dim >> 4;  // 8-wide chunks per half head
  const int ngrp = (n_heads + kRopeHG - 1) / kRopeHG;
  const int64_t per_tok = static_cast<int64_t>(ngrp) * cpp;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= tokens * per_tok) return;
  int64_t t, crow;
  int grp, c;
  if constexpr (WIDE) {
    t = idx / per_tok;
    const int rem = static_cast<int>(idx - t * per_tok);
    grp = rem / cpp;
    c = (rem - grp * cpp) * 8;
    crow = cos_per_token ? t : (t % seq_len);
  } else {
    const uint32_t i = static_cast<uint32_t>(idx), t32 = dv.per_tok.div(i);
    const uint32_t rem = i - t32 * static_cast<uint32_t>(per_tok);
    grp = static_cast<int>(dv.cpp.div(rem));
    c = static_cast<int>(rem - static_cast<uint32_t>(grp * cpp)) * 8;
    t = t32;
    crow = cos_per_token ? t : static_cast<int64_t>(t32 - dv.seq.div(t32) * static_cast<uint32_t>(seq_len));
  }
  const int half = head_dim >> 1;

  const T* cb = cosv + crow * head_dim + c;
  const T* sb = sinv + crow * head_dim + c;
  float c0[8], c1[8], s0[8], s1[8];
  Elem<T>::load8(cb, c0);
  Elem<T>::load8(cb + half, c1);
  Elem<T>::load8(sb, s0);
  Elem<T>::load8(sb + half, s1);
  const int h0 = grp * kRopeHG;
  const int nh = min(kRopeHG, n_heads - h0);
  T* base = qk + t * ld + static_cast<int64_t>(h0) * head_dim + c;
  typename Elem<T>::Raw r0[kRopeHG], r1[kRopeHG];
#pragma unroll
  for (int k = 0; k < kRopeHG; ++k)
    if (k < nh) {
      r0[k] = Elem<T>::ldraw(base + k * head_dim);
      r1[k] = Elem<T>::ldraw(base + k * head_dim + half);
    }
#pragma unroll
  for (int k = 0; k < kRopeHG; ++k) {
    if (k >= nh) break;
    float x0[8], x1[8], o0[8], o1[8];
    Elem<T>::unpack(r0[k], x0);
    Elem<T>::unpack(r1[k], x1);
#pragma unroll
    for (int j = 0; j < 8; ++j) rope_pair<T, BWD>(x0[j], x1[j], c0[j], c1[j], s0[j], s1[j], o0[j], o1[j]);
    Elem<T>::store8(base + k * head_dim, o0);
    Elem<T>::store8(base + k * head_dim + half, o1);
  }
}

// Streaming kernels: a block covers 256*kChunks consecutive 8-element chunks;
// thread t takes chunks t, t+256, ... (coalesced per step) and issues all its
// loads before computing.
template <typename T, bool WIDE>
__global__ __launch_bounds__(256) void k_swiglu_fwd(const T* __restrict__ g,
                                                    const T* __restrict__ u, int64_t ld_gu,
                                                    T* __restrict__ p, int64_t ld_p,
                                                    int64_t rows, int cols, FastDiv fd) {
  using Raw = typename Elem<T>::Raw;
  const int cpr = cols >> 3;
  const int64_t total = rows * cpr;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * (256 * kChunks) + threadIdx.x;
  Raw gr[kChunks], ur[kChunks];
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    const int64_t idx = first + 256 * k;
    if (idx < total) {
      int64_t r;
      int c;
      row_col<WIDE>(idx, cpr, fd, r, c);
      gr[k] = sw_load<T>(g + r * ld_gu + c);
      ur[k] = sw_load<T>(u + r * ld_gu + c);
    }
  }
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    const int64_t idx = first + 256 * k;
    if (idx >= total) break;
    int64_t r;
    int c;
    row_col<WIDE>(idx, cpr, fd, r, c);
    float gv[8], uv[8], o[8];
    Elem<T>::unpack(gr[k], gv);
    Elem<T>::unpack(ur[k], uv);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = Elem<T>::rnd(silu_f(gv[j])) * uv[j];
    Elem<T>::store8(p + r * ld_p + c, o);
  }
}

// With P, also p = silu(g) * u as k_swiglu_fwd rounds it (the stored silu(g)
// times u), written to p: a backward that did not keep the forward's product
// gets it from the pass that reads g and u anyway.  p may be dp itself (each
// thread reads its chunk of dp before it writes the same chunk of p), so
// neither is __restrict__.
template <typename T, bool WIDE, bool P>
__global__ __launch_bounds__(256) void k_swiglu_bwd(const T* dp, int64_t ld_dp,
                                                    const T* __restrict__ g,
                                                    const T* __restrict__ u, int64_t ld_gu,
                                                    T* __restrict__ dg, T* __restrict__ du,
                                                    int64_t ld_dgu, T* p, int64_t ld_p, int64_t rows, int cols,
                                                    FastDiv fd) {
  using Raw = typename Elem<T>::Raw;
  const int cpr = cols >> 3;
  const int64_t total = rows * cpr;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * (256 * kChunks) + threadIdx.x;
  Raw dr[kChunks], gr[kChunks], ur[kChunks];
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    const int64_t idx = first + 256 * k;
    if (idx < total) {
      int64_t r;
      int c;
      row_col<WIDE>(idx, cpr, fd, r, c);
      dr[k] = sw_load<T>(dp + r * ld_dp + c);
      gr[k] = sw_load<T>(g + r * ld_gu + c);
      ur[k] = sw_load<T>(u + r * ld_gu + c);
    }
  }
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    const int64_t idx = first + 256 * k;
    if (idx >= total) break;
    int64_t r;
    int c;
    row_col<WIDE>(idx, cpr, fd, r, c);
    float dv[8], gv[8], uv[8], og[8], ou[8], op[8];
    Elem<T>::unpack(dr[k], dv);
    Elem<T>::unpack(gr[k], gv);
    Elem<T>::unpack(ur[k], uv);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float sg = sigmoid_f(gv[j]);
      const float s = Elem<T>::rnd(gv[j] * sg);          // the stored silu(g) (= rnd(silu_f(g)))
      ou[j] = dv[j] * s;                                  // d(up)
      const float ds = Elem<T>::rnd(dv[j] * uv[j]);       // grad at silu output
      og[j] = ds * sg * (1.f + gv[j] * (1.f - sg));       // silu_backward
      if constexpr (P) op[j] = s * uv[j];                 // the forward's product
    }
    Elem<T>::store8(dg + r * ld_dgu + c, og);
    Elem<T>::store8(du + r * ld_dgu + c, ou);
    if constexpr (P) Elem<T>::store8(p + r * ld_p + c, op);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_add(const T* a, const T* b, T* out, int64_t n8) {
  using Raw = typename Elem<T>::Raw;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * (256 * kChunks) + threadIdx.x;
  Raw ar[kChunks], br[kChunks];
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    const int64_t i = first + 256 * k;
    if (i < n8) {
      ar[k] = Elem<T>::ldraw(a + i * 8);
      br[k] = Elem<T>::ldraw(b + i * 8);
    }
  }
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    const int64_t i = first + 256 * k;
    if (i >= n8) break;
    float av[8], bv[8];
    Elem<T>::unpack(ar[k], av);
    Elem<T>::unpack(br[k], bv);
#pragma unroll
    for (int j = 0; j < 8; ++j) av[j] += bv[j];
    Elem<T>::store8(out + i * 8, av);
  }
}

// out = to_dtype(x * scale[0]): the loss head's backward, which multiplies
// its saved input and weight gradients by the incoming gradient of the loss
// (a device scalar, so the host never waits for it).
template <typename T>
__global__ __launch_bounds__(256) void k_scale(const T* x, T* out, int64_t n8, const float* scale) {
  using Raw = typename Elem<T>::Raw;
  const float s = *scale;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * (256 * kChunks) + threadIdx.x;
  Raw xr[kChunks];
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    const int64_t i = first + 256 * k;
    if (i < n8) xr[k] = Elem<T>::ldraw(x + i * 8);
  }
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    const int64_t i = first + 256 * k;
    if (i >= n8) break;
    float v[8];
    Elem<T>::unpack(xr[k], v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= s;
    Elem<T>::store8(out + i * 8, v);
  }
}

inline unsigned blocks_for(int64_t threads) {
  return static_cast<unsigned>((threads + 255) / 256);
}

// Blocks for a streaming kernel over `chunks` 8-element chunks.
inline unsigned stream_blocks(int64_t chunks) {
  return static_cast<unsigned>((chunks + 256 * kChunks - 1) / (256 * kChunks));
}

inline bool ok_dtype(fh_dtype dt) { return dt == FH_BF16 || dt == FH_F32; }

template <bool BWD>
int rope_impl(fh_dtype dt, void* qk, int64_t ld, int64_t tokens, int64_t seq_len,
              int64_t n_heads, int64_t head_dim, const void* cosv, const void* sinv,
              int cos_per_token, hipStream_t s) {
  FH_REQUIRE(ok_dtype(dt), "rope: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(tokens >= 0 && n_heads >= 0, "rope: negative size");
  FH_REQUIRE(head_dim > 0 && head_dim % 16 == 0 && head_dim <= 512,
             "rope: head_dim must be a positive multiple of 16 (<= 512)");
  FH_REQUIRE(seq_len > 0, "rope: seq_len must be > 0");
  FH_REQUIRE(cos_per_token || tokens % seq_len == 0, "rope: tokens must be a multiple of seq_len");
  FH_REQUIRE(ld >= n_heads * head_dim && ld % 8 == 0, "rope: ld too small or not a multiple of 8");
  if (tokens == 0 || n_heads == 0) return FH_OK;
  FH_REQUIRE(qk && cosv && sinv, "rope: null pointer");
  FH_REQUIRE(aligned16(qk) && aligned16(cosv) && aligned16(sinv), "rope: pointers must be 16-byte aligned");
  const int64_t per_tok = ((n_heads + kRopeHG - 1) / kRopeHG) * (head_dim / 16);
  const int64_t threads = tokens * per_tok;
  const bool w64 = wide(threads) || seq_len >= (int64_t(1) << 32);
  const RopeDivs dv{FastDiv(static_cast<uint32_t>(per_tok)), FastDiv(static_cast<uint32_t>(head_dim / 16)),
                    FastDiv(static_cast<uint32_t>(w64 ? 1 : seq_len))};
  auto go = [&](auto tag, auto wide_c) {
    using T = decltype(tag);
    hipLaunchKernelGGL((k_rope<T, BWD, decltype(wide_c)::value>), dim3(blocks_for(threads)),
                       dim3(256), 0, s, static_cast<T*>(qk), ld, tokens, seq_len,
                       static_cast<int>(n_heads), static_cast<int>(head_dim),
                       static_cast<const T*>(cosv), static_cast<const T*>(sinv), cos_per_token, dv);
  };
  if (dt == FH_BF16) {
    if (w64) go(uint16_t{}, std::true_type{});
    else go(uint16_t{}, std::false_type{});
  } else {
    if (w64) go(float{}, std::true_type{});
    else go(float{}, std::false_type{});
  }
  return check_launch(BWD ? "fh_rope_bwd" : "fh_rope_fwd");
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" int fh_rope_fwd(fh_dtype dt, void* qk, int64_t ld, int64_t tokens, int64_t seq_len,
                           int64_t n_heads, int64_t head_dim, const void* cosv, const void* sinv,
                           int cos_per_token, hipStream_t stream) {
  return rope_impl<false>(dt, qk, ld, tokens, seq_len, n_heads, head_dim, cosv, sinv,
                          cos_per_token, stream);
}

extern "C" int fh_rope_bwd(fh_dtype dt, void* dqk, int64_t ld, int64_t tokens, int64_t seq_len,
                           int64_t n_heads, int64_t head_dim, const void* cosv, const void* sinv,
                           int cos_per_token, hipStream_t stream) {
  return rope_impl<true>(dt, dqk, ld, tokens, seq_len, n_heads, head_dim, cosv, sinv,
                         cos_per_token, stream);
}

extern "C" int fh_swiglu_fwd(fh_dtype dt, const void* g, const void* u, int64_t ld_gu, void* p,
                             int64_t ld_p, int64_t rows, int64_t cols, hipStream_t stream) {
  FH_REQUIRE(ok_dtype(dt), "swiglu_fwd: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0, "swiglu_fwd: cols must be a positive multiple of 8");
  FH_REQUIRE(ld_gu >= cols && ld_p >= cols && ld_gu % 8 == 0 && ld_p % 8 == 0,
             "swiglu_fwd: leading dims must be >= cols and multiples of 8");
  if (rows == 0) return FH_OK;
  FH_REQUIRE(g && u && p, "swiglu_fwd: null pointer");
  FH_REQUIRE(aligned16(g) && aligned16(u) && aligned16(p), "swiglu_fwd: pointers must be 16-byte aligned");
  const int64_t threads = rows * (cols / 8);
  const FastDiv fd(static_cast<uint32_t>(cols / 8));
  auto go = [&](auto tag, auto wide_c) {
    using T = decltype(tag);
    hipLaunchKernelGGL((k_swiglu_fwd<T, decltype(wide_c)::value>), dim3(stream_blocks(threads)),
                       dim3(256), 0, stream, static_cast<const T*>(g), static_cast<const T*>(u),
                       ld_gu, static_cast<T*>(p), ld_p, rows, static_cast<int>(cols), fd);
  };
  if (dt == FH_BF16) {
    if (wide(threads)) go(uint16_t{}, std::true_type{});
    else go(uint16_t{}, std::false_type{});
  } else {
    if (wide(threads)) go(float{}, std::true_type{});
    else go(float{}, std::false_type{});
  }
  return check_launch("fh_swiglu_fwd");
}

extern "C" int fh_swiglu_bwd(fh_dtype dt, const void* dp, int64_t ld_dp, const void* g,
                             const void* u, int64_t ld_gu, void* dg, void* du, int64_t ld_dgu,
                             void* p, int64_t ld_p, int64_t rows, int64_t cols, hipStream_t stream) {
  FH_REQUIRE(ok_dtype(dt), "swiglu_bwd: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0, "swiglu_bwd: cols must be a positive multiple of 8");
  FH_REQUIRE(ld_dp >= cols && ld_gu >= cols && ld_dgu >= cols && ld_dp % 8 == 0 &&
                 ld_gu % 8 == 0 && ld_dgu % 8 == 0,
             "swiglu_bwd: leading dims must be >= cols and multiples of 8");
  FH_REQUIRE(!p || (ld_p >= cols && ld_p % 8 == 0), "swiglu_bwd: ld_p must be >= cols and a multiple of 8");
  FH_REQUIRE(!p || p != dp || ld_p == ld_dp, "swiglu_bwd: p aliasing dp must share its leading dim");
  if (rows == 0) return FH_OK;
  FH_REQUIRE(dp && g && u && dg && du, "swiglu_bwd: null pointer");
  FH_REQUIRE(aligned16(dp) && aligned16(g) && aligned16(u) && aligned16(dg) && aligned16(du) &&
                 (!p || aligned16(p)),
             "swiglu_bwd: pointers must be 16-byte aligned");
  const int64_t threads = rows * (cols / 8);
  const FastDiv fd(static_cast<uint32_t>(cols / 8));
  auto go = [&](auto tag, auto wide_c, auto p_c) {
    using T = decltype(tag);
    hipLaunchKernelGGL((k_swiglu_bwd<T, decltype(wide_c)::value, decltype(p_c)::value>),
                       dim3(stream_blocks(threads)), dim3(256), 0, stream, static_cast<const T*>(dp), ld_dp,
                       static_cast<const T*>(g), static_cast<const T*>(u), ld_gu,
                       static_cast<T*>(dg), static_cast<T*>(du), ld_dgu, static_cast<T*>(p), ld_p, rows,
                       static_cast<int>(cols), fd);
  };
  auto with_p = [&](auto tag, auto wide_c) {
    if (p) go(tag, wide_c, std::true_type{});
    else go(tag, wide_c, std::false_type{});
  };
  if (dt == FH_BF16) {
    if (wide(threads)) with_p(uint16_t{}, std::true_type{});
    else with_p(uint16_t{}, std::false_type{});
  } else {
    if (wide(threads)) with_p(float{}, std::true_type{});
    else with_p(float{}, std::false_type{});
  }
  return check_launch("fh_swiglu_bwd");
}

extern "C" int fh_add(fh_dtype dt, const void* a, const void* b, void* out, int64_t n,
                      hipStream_t stream) {
  FH_REQUIRE(ok_dtype(dt), "add: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(n >= 0 && n % 8 == 0, "add: n must be a non-negative multiple of 8");
  if (n == 0) return FH_OK;
  FH_REQUIRE(a && b && out, "add: null pointer");
  FH_REQUIRE(aligned16(a) && aligned16(b) && aligned16(out), "add: pointers must be 16-byte aligned");
  if (dt == FH_BF16)
    hipLaunchKernelGGL((k_add<uint16_t>), dim3(stream_blocks(n / 8)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                       static_cast<uint16_t*>(out), n / 8);
  else
    hipLaunchKernelGGL((k_add<float>), dim3(stream_blocks(n / 8)), dim3(256), 0, stream,
                       static_cast<const float*>(a), static_cast<const float*>(b),
                       static_cast<float*>(out), n / 8);
  return check_launch("fh_add");
}

extern "C" int fh_scale(fh_dtype dt, const void* x, void* out, int64_t n, const float* scale,
                        hipStream_t stream) {
  FH_REQUIRE(ok_dtype(dt), "scale: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(n >= 0 && n % 8 == 0, "scale: n must be a non-negative multiple of 8");
  if (n == 0) return FH_OK;
  FH_REQUIRE(x && out && scale, "scale: null pointer");
  FH_REQUIRE(aligned16(x) && aligned16(out), "scale: pointers must be 16-byte aligned");
  if (dt == FH_BF16)
    hipLaunchKernelGGL((k_scale<uint16_t>), dim3(stream_blocks(n / 8)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<uint16_t*>(out), n / 8, scale);
  else
    hipLaunchKernelGGL((k_scale<float>), dim3(stream_blocks(n / 8)), dim3(256), 0, stream,
                       static_cast<const float*>(x), static_cast<float*>(out), n / 8, scale);
  return check_launch("fh_scale");
}
