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
#include "fh_common.hpp"

namespace fh {
namespace {

__device__ __forceinline__ float silu_f(float g) { return g / (1.f + expf(-g)); }
__device__ __forceinline__ float sigmoid_f(float g) { return 1.f / (1.f + expf(-g)); }

// One thread = 8 rotation pairs (i, i + d/2) of one head of one token.
template <typename T, bool BWD>
__global__ __launch_bounds__(256) void k_rope(T* __restrict__ qk, int64_t ld, int64_t tokens,
                                              int64_t seq_len, int n_heads, int head_dim,
                                              const T* __restrict__ cosv,
                                              const T* __restrict__ sinv, int cos_per_token) {
  const int cpp = head_dim >> 4;  // 8-wide chunks per half head
  const int64_t per_tok = static_cast<int64_t>(n_heads) * cpp;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= tokens * per_tok) return;
  const int64_t t = idx / per_tok;
  const int rem = static_cast<int>(idx - t * per_tok);
  const int hh = rem / cpp;
  const int c = (rem - hh * cpp) * 8;
  const int half = head_dim >> 1;
  const int64_t crow = cos_per_token ? t : (t % seq_len);

  T* p0 = qk + t * ld + static_cast<int64_t>(hh) * head_dim + c;
  T* p1 = p0 + half;
  const T* cb = cosv + crow * head_dim + c;
  const T* sb = sinv + crow * head_dim + c;
  float x0[8], x1[8], c0[8], c1[8], s0[8], s1[8];
  Elem<T>::load8(p0, x0);
  Elem<T>::load8(p1, x1);
  Elem<T>::load8(cb, c0);
  Elem<T>::load8(cb + half, c1);
  Elem<T>::load8(sb, s0);
  Elem<T>::load8(sb + half, s1);
  float o0[8], o1[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (!BWD) {
      // q*cos + rotate_half(q)*sin, rotate_half(q) = cat(-q[d/2:], q[:d/2])
      o0[j] = Elem<T>::rnd(Elem<T>::rnd(x0[j] * c0[j]) - Elem<T>::rnd(x1[j] * s0[j]));
      o1[j] = Elem<T>::rnd(Elem<T>::rnd(x1[j] * c1[j]) + Elem<T>::rnd(x0[j] * s1[j]));
    } else {
      // transpose of the rotation: grad*cos + rotate_half^T(grad*sin)
      o0[j] = Elem<T>::rnd(Elem<T>::rnd(x0[j] * c0[j]) + Elem<T>::rnd(x1[j] * s1[j]));
      o1[j] = Elem<T>::rnd(Elem<T>::rnd(x1[j] * c1[j]) - Elem<T>::rnd(x0[j] * s0[j]));
    }
  }
  Elem<T>::store8(p0, o0);
  Elem<T>::store8(p1, o1);
}

template <typename T>
__global__ __launch_bounds__(256) void k_swiglu_fwd(const T* __restrict__ g,
                                                    const T* __restrict__ u, int64_t ld_gu,
                                                    T* __restrict__ p, int64_t ld_p,
                                                    int64_t rows, int cols) {
  const int cpr = cols >> 3;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows * cpr) return;
  const int64_t r = idx / cpr;
  const int c = static_cast<int>(idx - r * cpr) * 8;
  float gv[8], uv[8], o[8];
  Elem<T>::load8(g + r * ld_gu + c, gv);
  Elem<T>::load8(u + r * ld_gu + c, uv);
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = Elem<T>::rnd(silu_f(gv[j])) * uv[j];
  Elem<T>::store8(p + r * ld_p + c, o);
}

template <typename T>
__global__ __launch_bounds__(256) void k_swiglu_bwd(const T* __restrict__ dp, int64_t ld_dp,
                                                    const T* __restrict__ g,
                                                    const T* __restrict__ u, int64_t ld_gu,
                                                    T* __restrict__ dg, T* __restrict__ du,
                                                    int64_t ld_dgu, int64_t rows, int cols) {
  const int cpr = cols >> 3;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows * cpr) return;
  const int64_t r = idx / cpr;
  const int c = static_cast<int>(idx - r * cpr) * 8;
  float dv[8], gv[8], uv[8], og[8], ou[8];
  Elem<T>::load8(dp + r * ld_dp + c, dv);
  Elem<T>::load8(g + r * ld_gu + c, gv);
  Elem<T>::load8(u + r * ld_gu + c, uv);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float sg = sigmoid_f(gv[j]);
    const float s = Elem<T>::rnd(gv[j] * sg);          // the stored silu(g)
    ou[j] = dv[j] * s;                                  // d(up)
    const float ds = Elem<T>::rnd(dv[j] * uv[j]);       // grad at silu output
    og[j] = ds * sg * (1.f + gv[j] * (1.f - sg));       // silu_backward
  }
  Elem<T>::store8(dg + r * ld_dgu + c, og);
  Elem<T>::store8(du + r * ld_dgu + c, ou);
}

template <typename T>
__global__ __launch_bounds__(256) void k_add(const T* a, const T* b, T* out, int64_t n8) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n8) return;
  float av[8], bv[8];
  Elem<T>::load8(a + i * 8, av);
  Elem<T>::load8(b + i * 8, bv);
#pragma unroll
  for (int j = 0; j < 8; ++j) av[j] += bv[j];
  Elem<T>::store8(out + i * 8, av);
}

inline unsigned blocks_for(int64_t threads) {
  return static_cast<unsigned>((threads + 255) / 256);
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
  const int64_t threads = tokens * n_heads * (head_dim / 16);
  if (dt == FH_BF16)
    hipLaunchKernelGGL((k_rope<uint16_t, BWD>), dim3(blocks_for(threads)), dim3(256), 0, s,
                       static_cast<uint16_t*>(qk), ld, tokens, seq_len, static_cast<int>(n_heads),
                       static_cast<int>(head_dim), static_cast<const uint16_t*>(cosv),
                       static_cast<const uint16_t*>(sinv), cos_per_token);
  else
    hipLaunchKernelGGL((k_rope<float, BWD>), dim3(blocks_for(threads)), dim3(256), 0, s,
                       static_cast<float*>(qk), ld, tokens, seq_len, static_cast<int>(n_heads),
                       static_cast<int>(head_dim), static_cast<const float*>(cosv),
                       static_cast<const float*>(sinv), cos_per_token);
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
  if (dt == FH_BF16)
    hipLaunchKernelGGL((k_swiglu_fwd<uint16_t>), dim3(blocks_for(threads)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u), ld_gu,
                       static_cast<uint16_t*>(p), ld_p, rows, static_cast<int>(cols));
  else
    hipLaunchKernelGGL((k_swiglu_fwd<float>), dim3(blocks_for(threads)), dim3(256), 0, stream,
                       static_cast<const float*>(g), static_cast<const float*>(u), ld_gu,
                       static_cast<float*>(p), ld_p, rows, static_cast<int>(cols));
  return check_launch("fh_swiglu_fwd");
}

extern "C" int fh_swiglu_bwd(fh_dtype dt, const void* dp, int64_t ld_dp, const void* g,
                             const void* u, int64_t ld_gu, void* dg, void* du, int64_t ld_dgu,
                             int64_t rows, int64_t cols, hipStream_t stream) {
  FH_REQUIRE(ok_dtype(dt), "swiglu_bwd: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0, "swiglu_bwd: cols must be a positive multiple of 8");
  FH_REQUIRE(ld_dp >= cols && ld_gu >= cols && ld_dgu >= cols && ld_dp % 8 == 0 &&
                 ld_gu % 8 == 0 && ld_dgu % 8 == 0,
             "swiglu_bwd: leading dims must be >= cols and multiples of 8");
  if (rows == 0) return FH_OK;
  FH_REQUIRE(dp && g && u && dg && du, "swiglu_bwd: null pointer");
  FH_REQUIRE(aligned16(dp) && aligned16(g) && aligned16(u) && aligned16(dg) && aligned16(du),
             "swiglu_bwd: pointers must be 16-byte aligned");
  const int64_t threads = rows * (cols / 8);
  if (dt == FH_BF16)
    hipLaunchKernelGGL((k_swiglu_bwd<uint16_t>), dim3(blocks_for(threads)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(dp), ld_dp, static_cast<const uint16_t*>(g),
                       static_cast<const uint16_t*>(u), ld_gu, static_cast<uint16_t*>(dg),
                       static_cast<uint16_t*>(du), ld_dgu, rows, static_cast<int>(cols));
  else
    hipLaunchKernelGGL((k_swiglu_bwd<float>), dim3(blocks_for(threads)), dim3(256), 0, stream,
                       static_cast<const float*>(dp), ld_dp, static_cast<const float*>(g),
                       static_cast<const float*>(u), ld_gu, static_cast<float*>(dg),
                       static_cast<float*>(du), ld_dgu, rows, static_cast<int>(cols));
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
    hipLaunchKernelGGL((k_add<uint16_t>), dim3(blocks_for(n / 8)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                       static_cast<uint16_t*>(out), n / 8);
  else
    hipLaunchKernelGGL((k_add<float>), dim3(blocks_for(n / 8)), dim3(256), 0, stream,
                       static_cast<const float*>(a), static_cast<const float*>(b),
                       static_cast<float*>(out), n / 8);
  return check_launch("fh_add");
}
