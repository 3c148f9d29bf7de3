// Causal GQA flash attention, forward and backward, for gfx950.
//
// Replaces F.scaled_dot_product_attention(q, k, v, is_causal=True,
// enable_gqa=True, scale=head_dim^-0.5) as called by sdpa_attention_forward
// (transformers 5.15.0 integrations/sdpa_attention.py:79-166) from
// LlamaAttention.forward (models/llama/modeling_llama.py:235-281), and its
// autograd backward.  Query head h reads kv head h / (n_heads / n_kv_heads)
// (repeat_kv, modeling_llama.py:179-188).
//
// Layout: token-major.  Row t = b*S + s of q/k/v/o holds all heads of one
// token (head h at columns h*HD..h*HD+HD-1), so q, k, v are column ranges of
// the layer's fused [T, Hq+2Hkv] projection output and o feeds the o_proj GEMM
// directly; no transposes ever touch HBM.
//
// bf16 kernels use v_mfma_f32_32x32x16_bf16.  Lane i of an MFMA operand holds
// row/col i%32 and K-slice 8*(i/32)..+7; lane i of the fp32 accumulator holds
// column i%32 and rows 8*(j/4) + 4*(i/32) + j%4, j = 0..15.  The softmax is
// formed on S^T (keys x queries) so each lane owns one query: row max / sum are
// in-lane plus one exchange with lane i^32, rescaling the output is a per-lane
// scalar, and P^T feeds the next MFMA straight from registers.  That P operand
// carries its K index (the key) in the permuted order {4h..4h+3, 8+4h..8+4h+3}
// (h = i/32) of the accumulator layout; the matching operand is fetched with
// two ds_read_b64_tr_b16 transpose reads in exactly that order.
//
// LDS tiles are [rows x HD] bf16 without padding, XOR-swizzled in 16-byte
// chunks: chunk c of row r is stored at chunk position c ^ swz(r).  Operands
// read a tile in two patterns, (a) ds_read_b128 of one chunk from 16
// consecutive rows and (b) ds_read_b64_tr_b16 of 4 consecutive chunks from 4
// consecutive rows (first row a multiple of 4) across 32 lanes; swz() maps
// both onto the 16 distinct 4-bank groups of one LDS cycle, so neither has
// bank conflicts.  A read address is a per-lane constant XOR a compile-time
// constant, plus an immediate offset.
#include <math.h>

#include <type_traits>

#include "fh_common.hpp"
#include "fh_mfma.hpp"

namespace fh {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// The forward keeps a stale running maximum until a block's maximum exceeds it
// by more than this (log2 units): the softmax weights then stay <= 2^8, and
// the output rescale runs only when the maximum really grows.
constexpr float kRescaleSlack = 8.f;

// 2^x on the transcendental unit (v_exp_f32).  Denormal results flush to
// zero, which is harmless for softmax weights.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// max over lanes i and i^32 (v_permlane32_swap exchanges the two row halves).
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// 8 consecutive bf16 from global memory.
__device__ __forceinline__ bf16x8 ld_frag(const uint16_t* p) {
  return as_bf16x8(*reinterpret_cast<const uint4*>(p));
}

// Accumulator entries j0..j0+7 rounded to bf16 as an MFMA operand.
__device__ __forceinline__ bf16x8 pack_frag(const f32x16& acc, int j0) {
  return as_bf16x8(make_uint4(pk_bf16(acc[j0 + 0], acc[j0 + 1]), pk_bf16(acc[j0 + 2], acc[j0 + 3]),
                              pk_bf16(acc[j0 + 4], acc[j0 + 5]), pk_bf16(acc[j0 + 6], acc[j0 + 7])));
}

// XCD-aware block order.  Workgroup L = blockIdx.x + gridDim.x*blockIdx.y is
// dispatched to XCD L % 8 (8 XCDs, each with its own L2).  Grids here are
// (work items along x, heads along y) with causal work varying along x, so the
// identity mapping gives XCD k only the x == k (mod 8) items of every head: an
// up to 2.4x imbalance between XCDs at 16 items per head.  This maps XCD k's
// j-th workgroup to head y = k*(gridDim.y/8) + j % (gridDim.y/8) and rank
// x = j / (gridDim.y/8): every XCD covers all x of its own contiguous set of
// heads (balanced work; one head's K/V/Q/dO stay in one L2), ranks in order
// (rank 0 = dispatched first).  Needs gridDim.y % 8 == 0, else identity.
struct XcdOrder {
  int rank, y;
};
__device__ __forceinline__ XcdOrder xcd_order() {
  const int nx = gridDim.x, ny = gridDim.y;
  if (ny % 8 != 0) return {static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y)};
  const int L = blockIdx.x + nx * blockIdx.y;
  const int xcd = L & 7, j = L >> 3, nyx = ny >> 3;
  return {j / nyx, xcd * nyx + j % nyx};
}

// Stores a transposed accumulator tile (rows = head dims d, column = this
// lane's token) scaled by `mul` into one token-major output row.
template <int HD>
__device__ __forceinline__ void store_rows_T(uint16_t* out_row, const f32x16 (&acc)[HD / 32],
                                             float mul, int hl) {
#pragma unroll
  for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint2 w;
      w.x = pk_bf16(acc[dt][4 * g] * mul, acc[dt][4 * g + 1] * mul);
      w.y = pk_bf16(acc[dt][4 * g + 2] * mul, acc[dt][4 * g + 3] * mul);
      *reinterpret_cast<uint2*>(out_row + dt * 32 + 8 * g + 4 * hl) = w;
    }
}

// Rotary tables of the RoPE backward fused into the dQ and dK stores:
// cos / sin rows of head_dim elements in the gradients' dtype, one row per
// position (per_token == 0) or per token; cos == null means plain stores.
template <typename T>
struct RopeRows {
  const T* cos;
  const T* sin;
  int per_token;
  // Row of position `pos` of the sequence whose first token is row tok0.
  __device__ __forceinline__ int64_t row(int64_t tok0, int pos) const { return per_token ? tok0 + pos : pos; }
};

__device__ __forceinline__ void unpack4_bf16(uint2 w, float (&v)[4]) {
  v[0] = __uint_as_float(w.x << 16);
  v[1] = __uint_as_float(w.x & 0xffff0000u);
  v[2] = __uint_as_float(w.y << 16);
  v[3] = __uint_as_float(w.y & 0xffff0000u);
}

// store_rows_T followed by the RoPE backward of the stored row: with
// x = bf16(acc * mul) it writes rope_pair<bf16, backward> of (x[d], x[d+HD/2])
// -- bit for bit what the plain store and a separate rope backward over the row
// give.  cs / sn point at this token's cos / sin row.  A lane holds dims
// dt*32 + 8g + 4hl + (0..3) of its token, so both halves of every pair are in
// the lane: the partner of (dt, g) is (dt + ND/2, g) for HD >= 64 and
// (dt, g + 2) for HD == 32.
template <int HD>
__device__ __forceinline__ void store_rows_T_rope(uint16_t* out_row, const f32x16 (&acc)[HD / 32], float mul,
                                                  int hl, const uint16_t* cs, const uint16_t* sn) {
  constexpr int ND = HD / 32, H2 = HD / 2;
#pragma unroll
  for (int dt = 0; dt < ND; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (dt * 32 + 8 * g >= H2) continue;  // upper half: written with its partner
      const int dt2 = HD == 32 ? dt : dt + ND / 2, g2 = HD == 32 ? g + 2 : g;
      const int d0 = dt * 32 + 8 * g + 4 * hl, d1 = d0 + H2;
      float c0[4], c1[4], s0[4], s1[4], o0[4], o1[4];
      unpack4_bf16(*reinterpret_cast<const uint2*>(cs + d0), c0);
      unpack4_bf16(*reinterpret_cast<const uint2*>(cs + d1), c1);
      unpack4_bf16(*reinterpret_cast<const uint2*>(sn + d0), s0);
      unpack4_bf16(*reinterpret_cast<const uint2*>(sn + d1), s1);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        rope_pair<uint16_t, true>(round_bf(acc[dt][4 * g + i] * mul), round_bf(acc[dt2][4 * g2 + i] * mul), c0[i],
                                  c1[i], s0[i], s1[i], o0[i], o1[i]);
      *reinterpret_cast<uint2*>(out_row + d0) = make_uint2(pk_bf16(o0[0], o0[1]), pk_bf16(o0[2], o0[3]));
      *reinterpret_cast<uint2*>(out_row + d1) = make_uint2(pk_bf16(o1[0], o1[1]), pk_bf16(o1[2], o1[3]));
    }
}

// The dQ / dK store of token `pos` (row tok0 + pos), rotated when rope.cos is set.
template <int HD>
__device__ __forceinline__ void store_grad_row(uint16_t* out_row, const f32x16 (&acc)[HD / 32], float mul, int hl,
                                               const RopeRows<uint16_t>& rope, int64_t tok0, int pos) {
  if (rope.cos) {
    const int64_t r = rope.row(tok0, pos) * HD;
    store_rows_T_rope<HD>(out_row, acc, mul, hl, rope.cos + r, rope.sin + r);
  } else {
    store_rows_T<HD>(out_row, acc, mul, hl);
  }
}

// The forward rotation of one query row's fragments as ld_frag loads them
// (fragment s of the lane holds dims 16s + 8hl .. +7, so the pair partner of
// fragment s is fragment s + HD/32, in the same lane), with the arithmetic of
// the standalone rope kernel; out_row (nullable) receives the rotated row.
template <int HD>
__device__ __forceinline__ void rope_q_frags(bf16x8 (&qf)[HD / 16], const uint16_t* cs, const uint16_t* sn,
                                             int hl, uint16_t* out_row) {
  constexpr int H2 = HD / 32;
#pragma unroll
  for (int s = 0; s < H2; ++s) {
    const int d0 = 16 * s + 8 * hl, d1 = d0 + HD / 2;
    float x0[8], x1[8], c0[8], c1[8], s0[8], s1[8], o0[8], o1[8];
    Elem<uint16_t>::unpack(__builtin_bit_cast(uint4, qf[s]), x0);
    Elem<uint16_t>::unpack(__builtin_bit_cast(uint4, qf[s + H2]), x1);
    Elem<uint16_t>::load8(cs + d0, c0);
    Elem<uint16_t>::load8(cs + d1, c1);
    Elem<uint16_t>::load8(sn + d0, s0);
    Elem<uint16_t>::load8(sn + d1, s1);
#pragma unroll
    for (int e = 0; e < 8; ++e) rope_pair<uint16_t, false>(x0[e], x1[e], c0[e], c1[e], s0[e], s1[e], o0[e], o1[e]);
    const uint4 p0 = Elem<uint16_t>::pack(o0), p1 = Elem<uint16_t>::pack(o1);
    qf[s] = as_bf16x8(p0);
    qf[s + H2] = as_bf16x8(p1);
    if (out_row) {
      *reinterpret_cast<uint4*>(out_row + d0) = p0;
      *reinterpret_cast<uint4*>(out_row + d1) = p1;
    }
  }
}

// ------------------------------------------------------------ forward (bf16)
// Block = 4 waves x (32*QT) queries of one (batch, head); loop over 64-key
// blocks, double-buffered in LDS: the next block's K/V are loaded straight
// into the other LDS stage while the current one is multiplied (no registers
// hold them in flight); one barrier per block.  QT query tiles per wave: QT = 2 would
// let every K/V fragment read from LDS feed two MFMAs, but its registers cost
// a wave of occupancy and it measured slower at head_dim 64 (342 vs 308 us at
// the TinyLlama shape), so QT = 1.  Heaviest (latest) query blocks first.
// With GQA (two query heads per kv head) a block of HPB = 2 x 4 waves takes the
// same query rows of two query heads, which read the same K/V tiles: each tile
// loaded into LDS feeds twice the MFMAs (TinyLlama 199 -> 190 us, rotated q
// 205-215 -> 203 us; Llama-3 slice 541-546 -> 506 us; bit-identical output).
template <int HD>
struct FwdTiles {
  static constexpr int QT = 1;
};

// The key-block loop of the forward and dQ kernels (4 waves): block kb + 1's
// K and V go straight into the other LDS stage (dma_tile) while
// body(kb, K, V) multiplies block kb; each wave waits for its own loads
// before the barrier that ends the block.  The two stages are separate
// arrays and the loop is unrolled by two, so every access names its stage
// and the compiler can tell that the loads into one stage do not alias the
// reads of the other (it would otherwise wait for them before every read).
// FAST: per-lane load addresses computed once (TileDma: no vector address
// arithmetic per load, 4-8 more registers); the dQ kernel, at the edge of an
// occupancy step, computes them per load instead (dma_tile).
// pre() runs once after block 0's loads are issued, before they are waited
// for (the kernel's own loads then overlap them).
template <int BN, int HD, bool FAST, int NW, class Body, class Pre>
__device__ __forceinline__ void kv_block_loop(const uint16_t* kb_ptr, int64_t ldk, const uint16_t* vb_ptr,
                                              int64_t ldv, int nkb, int S, char* sk0, char* sk1, char* sv0,
                                              char* sv1, int wave, int lane, Body&& body, Pre&& pre) {
  TileDma<BN, HD, NW> dk, dv;
  dk.init(ldk, wave, lane);
  dv.init(ldv, wave, lane);
  auto load = [&](int r0, char* KN, char* VN) __attribute__((always_inline)) {
    if constexpr (FAST) {
      dk.load(kb_ptr, ldk, r0, S - 1, KN, wave, lane);
      dv.load(vb_ptr, ldv, r0, S - 1, VN, wave, lane);
    } else {
      dk.load_asm(kb_ptr, ldk, r0, S - 1, KN, wave, lane);
      dv.load_asm(vb_ptr, ldv, r0, S - 1, VN, wave, lane);
    }
  };
  load(0, sk0, sv0);
  pre();
  wait_loads();
  __syncthreads();
  auto step = [&](int kb, const char* K, const char* V, char* KN, char* VN) __attribute__((always_inline)) {
    if (kb + 1 < nkb) load((kb + 1) * BN, KN, VN);
    if (kb < nkb) body(kb, K, V);
    wait_loads();
    __syncthreads();
  };
  for (int kb = 0; kb < nkb; kb += 2) {
    step(kb, sk0, sv0, sk1, sv1);
    step(kb + 1, sk1, sv1, sk0, sv0);
  }
}

// kv_block_loop with three LDS stages (the forward): block kb + 2's K and V are
// loaded while block kb is multiplied, so each block's loads have two blocks'
// time to land.  The barrier that ends a block waits for block kb + 1's loads
// only (vmcnt: the vector memory counter retires a wave's loads in issue
// order, and block kb + 2's loads are the wave's last ones), not for the ones
// still in flight into the third stage.
template <int BN, int HD, int NW, class Body, class Pre>
__device__ __forceinline__ void kv_block_loop3(const uint16_t* kb_ptr, int64_t ldk, const uint16_t* vb_ptr,
                                               int64_t ldv, int nkb, int S, char* sk0, char* sk1, char* sk2,
                                               char* sv0, char* sv1, char* sv2, int wave, int lane, Body&& body,
                                               Pre&& pre) {
  using Dma = TileDma<BN, HD, NW>;
  Dma dk, dv;
  dk.init(ldk, wave, lane);
  dv.init(ldv, wave, lane);
  // Loads this wave issues per block (K and V alike, in either of TileDma's paths).
  int per_wave = 0;
#pragma unroll
  for (int i = 0; i < Dma::PER; ++i) per_wave += (i * NW + wave < Dma::RUNS) ? 1 : 0;
  // The loads as inline asm (load_asm): the compiler, which cannot see the
  // waits below retire a stage's loads, would otherwise wait for every load
  // in flight before reading a stage.
  auto load = [&](int r0, char* KN, char* VN) __attribute__((always_inline)) {
    dk.load_asm(kb_ptr, ldk, r0, S - 1, KN, wave, lane);
    dv.load_asm(vb_ptr, ldv, r0, S - 1, VN, wave, lane);
  };
  load(0, sk0, sv0);
  if (nkb > 1) load(BN, sk1, sv1);
  pre();
  // vmcnt(0) as the builtin, which the compiler's own wait placement sees: it
  // then knows pre()'s loads have landed and puts no waits for them in the loop.
  __builtin_amdgcn_s_waitcnt(0x0f70);
  __syncthreads();
  auto step = [&](int kb, const char* K, const char* V, char* KN, char* VN) __attribute__((always_inline)) {
    const bool ahead = kb + 2 < nkb;
    if (ahead) load((kb + 2) * BN, KN, VN);
    if (kb < nkb) body(kb, K, V);
    if (ahead && per_wave == 1) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else if (ahead && per_wave == 2) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else wait_loads();
    lds_barrier();
  };
  for (int kb = 0; kb < nkb; kb += 3) {
    step(kb, sk0, sv0, sk2, sv2);
    step(kb + 1, sk1, sv1, sk0, sv0);
    step(kb + 2, sk2, sv2, sk1, sv1);
  }
}

// One 64-key block of the forward for one wave: raw scores from K (LDS),
// online softmax update of (m, l, oacc), then oacc += P V (V from LDS).
template <int HD, int QT>
__device__ __forceinline__ void fwd_block(const char* K, const char* V, const bf16x8 (&qf)[QT][HD / 16],
                                          f32x16 (&oacc)[QT][HD / 32], float (&m)[QT], float (&l)[QT],
                                          int a_off, int b0, int b8, int k0, int qw, int l32, int hl,
                                          int S, float scale_log2) {
  constexpr int BN = 64, NS = HD / 16, ND = HD / 32;
  f32x16 x[BN / 32][QT];  // raw scores S^T, rows = keys, column = query
  __builtin_amdgcn_iglp_opt(0);  // LDS reads interleaved with MFMAs (head_dim 128: -3%)
#pragma unroll
  for (int t = 0; t < BN / 32; ++t) {
#pragma unroll
    for (int u = 0; u < QT; ++u) x[t][u] = zero16();
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const bf16x8 a = lds_frag<HD>(K, a_off, 32 * t, s);
#pragma unroll
      for (int u = 0; u < QT; ++u) x[t][u] = mfma(a, qf[u][s], x[t][u]);
    }
  }
  const bool need_mask = (k0 + BN - 1 > qw) || (k0 + BN > S);
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    const int qi = qw + 32 * u + l32;
    float mloc = -INFINITY;
    if (need_mask) {  // diagonal or ragged block
      // key = k0 + 32t + acc_row(j, hl) is masked when key > qi or key >= S,
      // i.e. when its compile-time part 32t + acc_row(j, 0) exceeds lim.
      const int lim = min(qi, S - 1) - k0 - 4 * hl;
#pragma unroll
      for (int t = 0; t < BN / 32; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          x[t][u][j] = 32 * t + acc_row(j, 0) > lim ? -INFINITY : x[t][u][j];
          mloc = fmaxf(mloc, x[t][u][j]);
        }
    } else {
#pragma unroll
      for (int t = 0; t < BN / 32; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) mloc = fmaxf(mloc, x[t][u][j]);
    }
    mloc = xor32_max(mloc) * scale_log2;
    if (wave_any(mloc > m[u] + kRescaleSlack)) {
      const float mnew = fmaxf(m[u], mloc);
      const float alpha = fast_exp2(m[u] - mnew);
      m[u] = mnew;
      l[u] *= alpha;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) oacc[u][dt][j] *= alpha;
    }
    const float nm = -m[u];
#pragma unroll
    for (int t = 0; t < BN / 32; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) x[t][u][j] = fast_exp2(fmaf(x[t][u][j], scale_log2, nm));
  }
  // The row sums add the bf16 weights that P V multiplies (v_dot2 on the
  // packed fragments), so the normalisation matches the weights used.
  float lsum[QT];
#pragma unroll
  for (int u = 0; u < QT; ++u) lsum[u] = 0.f;
#pragma unroll
  for (int s = 0; s < BN / 16; ++s) {
    bf16x8 pf[QT];
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      pf[u] = pack_frag(x[s >> 1][u], 8 * (s & 1));
      lsum[u] = sum_bf16x8(pf[u], lsum[u]);
    }
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      const bf16x8 a = lds_frag_tr<HD>(V, b0, b8, 16 * s, dt);
#pragma unroll
      for (int u = 0; u < QT; ++u) oacc[u][dt] = mfma(a, pf[u], oacc[u][dt]);
    }
  }
#pragma unroll
  for (int u = 0; u < QT; ++u) l[u] += lsum[u];
}

// q and qout may be the same buffer (the rotated q written back in place), so
// neither is __restrict__: a lane stores only elements it has loaded.
template <int HD, int HPB>
__global__ __launch_bounds__(256 * HPB) __attribute__((amdgpu_waves_per_eu(2))) void k_attn_fwd(
    const uint16_t* q, int64_t ldq, const uint16_t* __restrict__ k, int64_t ldk,
    const uint16_t* __restrict__ v, int64_t ldv, uint16_t* __restrict__ o, int64_t ldo,
    float* __restrict__ lse, int S, int nh, int group, float scale_log2, RopeRows<uint16_t> rope,
    uint16_t* qout, int64_t ldqo) {
  constexpr int QT = FwdTiles<HD>::QT;
  constexpr int BM = 4 * 32 * QT, BN = 64, NS = HD / 16, ND = HD / 32, TILE = BN * 2 * HD;
  // Three K/V stages up to head_dim 64 (48 KB); at 128 three stages (96 KB)
  // would leave room for one workgroup per CU, so two.
  constexpr int STAGES = HD <= 64 ? 3 : 2, TILE3 = STAGES == 3 ? TILE : 16;
  __shared__ __align__(16) char sk0[TILE], sk1[TILE], sk2[TILE3], sv0[TILE], sv1[TILE], sv2[TILE3];
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const XcdOrder ord = xcd_order();
  const int nhb = nh / HPB, bg = ord.y, b = bg / nhb;
  const int h = (bg - b * nhb) * HPB + (wave >> 2), kvh = h / group, bh = b * nh + h;
  const int q0 = (gridDim.x - 1 - ord.rank) * BM;  // heaviest (latest) query blocks first
  const int qw = q0 + (wave & 3) * 32 * QT;  // first query of this wave
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  int a_off = lane_off_a<HD>(lane);
  int b0 = lane_off_b<HD>(lane, 0), b8 = lane_off_b<HD>(lane, 8);

  // Q fragments: loaded (and rotated) while the first K/V block is in flight.
  bf16x8 qf[QT][NS];
  auto load_q = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < QT; ++u) {
      const int qi = qw + 32 * u + l32;
      const uint16_t* qrow = q + (tok0 + qi) * ldq + static_cast<int64_t>(h) * HD + 8 * hl;
#pragma unroll
      for (int s = 0; s < NS; ++s)
        qf[u][s] = qi < S ? ld_frag(qrow + 16 * s) : as_bf16x8(make_uint4(0, 0, 0, 0));
      if (rope.cos && qi < S) {  // q rotated on load (RoPE forward), optionally written back
        const int64_t r = rope.row(tok0, qi) * HD;
        rope_q_frags<HD>(qf[u], rope.cos + r, rope.sin + r, hl,
                         qout ? qout + (tok0 + qi) * ldqo + static_cast<int64_t>(h) * HD : nullptr);
      }
    }
  };
  f32x16 oacc[QT][ND];
  float m[QT], l[QT];  // running max (log2 units) and sum of weights per query tile
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    m[u] = -INFINITY;
    l[u] = 0.f;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) oacc[u][dt] = zero16();
  }

  const int kend = min(S, q0 + BM);
  const int nkb = (kend + BN - 1) / BN;
  const uint16_t* kb_ptr = k + tok0 * ldk + static_cast<int64_t>(kvh) * HD;
  const uint16_t* vb_ptr = v + tok0 * ldv + static_cast<int64_t>(kvh) * HD;
  auto body = [&](int kb, const char* K, const char* V) __attribute__((always_inline)) {
    refresh_offsets(a_off, b0, b8);
    const int k0 = kb * BN;
    if (k0 <= qw + 32 * QT - 1)  // some key of the block precedes some query of the wave
      fwd_block<HD, QT>(K, V, qf, oacc, m, l, a_off, b0, b8, k0, qw, l32, hl, S, scale_log2);
  };
  if constexpr (STAGES == 3)
    kv_block_loop3<BN, HD, 4 * HPB>(kb_ptr, ldk, vb_ptr, ldv, nkb, S, sk0, sk1, sk2, sv0, sv1, sv2, wave, lane,
                                    body, load_q);
  else
    kv_block_loop<BN, HD, true, 4 * HPB>(kb_ptr, ldk, vb_ptr, ldv, nkb, S, sk0, sk1, sv0, sv1, wave, lane, body,
                                         load_q);
#pragma unroll
  for (int u = 0; u < QT; ++u) {
    const int qi = qw + 32 * u + l32;
    const float lt = xor32_sum(l[u]);
    if (qi < S) {
      store_rows_T<HD>(o + (tok0 + qi) * ldo + static_cast<int64_t>(h) * HD, oacc[u], 1.f / lt, hl);
      if (lse != nullptr && hl == 0) lse[static_cast<int64_t>(bh) * S + qi] = (m[u] + log2f(lt)) * kLn2;
    }
  }
}

// --------------------------------------- backward: delta = rowsum(dO*O), fp32
template <typename T>
__global__ __launch_bounds__(256) void k_attn_delta(const T* __restrict__ o, int64_t ldo,
                                                    const T* __restrict__ dO, int64_t lddo,
                                                    float* __restrict__ delta, int S, int nh,
                                                    int hd, int64_t tokens) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= tokens * nh) return;
  const int64_t t = idx / nh;
  const int h = static_cast<int>(idx - t * nh);
  const T* orow = o + t * ldo + static_cast<int64_t>(h) * hd;
  const T* grow = dO + t * lddo + static_cast<int64_t>(h) * hd;
  float acc = 0.f;
  for (int d = 0; d < hd; d += 8) {
    float a[8], g[8];
    Elem<T>::load8(orow + d, a);
    Elem<T>::load8(grow + d, g);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc = fmaf(a[j], g[j], acc);
  }
  const int64_t b = t / S;
  const int s = static_cast<int>(t - b * S);
  delta[(b * nh + h) * S + s] = acc;
}

// ------------------------------------------------------- backward: dQ (bf16)
// Same tiling as the forward with one 32-query tile per wave:
//   S^T = K Q^T, P^T = exp(S^T - lse), dP^T = V dO^T,
//   dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T, dQ = scale * dQ.
// The prologue also forms delta = rowsum(dO * O) of its queries (the lane
// holds half of each row; one exchange with lane i^32 completes it) and
// stores it for the dK/dV kernel, which runs next on the same stream.
// One 64-key block of the dQ kernel for one wave (query qi = qw + lane % 32).
template <int HD>
__device__ __forceinline__ void dq_block(const char* K, const char* V, const bf16x8 (&qf)[HD / 16],
                                         const bf16x8 (&gf)[HD / 16], f32x16 (&dqacc)[HD / 32], float nlse2,
                                         float dl, int a_off, int b0, int b8, int k0, int qw, int qi, int hl,
                                         int S, float scale_log2) {
  constexpr int BN = 64, NS = HD / 16, ND = HD / 32;
  const bool need_mask = (k0 + BN - 1 > qw) || (k0 + BN > S);
#pragma unroll
  for (int t = 0; t < BN / 32; ++t) {
    f32x16 x = zero16(), y = zero16();  // S^T, dP^T
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      x = mfma(lds_frag<HD>(K, a_off, 32 * t, s), qf[s], x);
      y = mfma(lds_frag<HD>(V, a_off, 32 * t, s), gf[s], y);
    }
    if (need_mask) {
      // key = k0 + 32t + acc_row(j, hl) is dead when key > qi or key >= S.
      const int lim = min(qi, S - 1) - k0 - 32 * t - 4 * hl;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float p = fast_exp2(fmaf(x[j], scale_log2, nlse2));
        x[j] = acc_row(j, 0) > lim ? 0.f : p * (y[j] - dl);  // dS^T
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) x[j] = fast_exp2(fmaf(x[j], scale_log2, nlse2)) * (y[j] - dl);
    }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const bf16x8 df = pack_frag(x, 8 * s2);
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
        dqacc[dt] = mfma(lds_frag_tr<HD>(K, b0, b8, 32 * t + 16 * s2, dt), df, dqacc[dt]);
    }
  }
}

template <int HD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_attn_bwd_dq(
    const uint16_t* __restrict__ q, int64_t ldq, const uint16_t* __restrict__ k, int64_t ldk,
    const uint16_t* __restrict__ v, int64_t ldv, const uint16_t* __restrict__ o, int64_t ldo,
    const uint16_t* __restrict__ dO, int64_t lddo, const float* __restrict__ lse,
    float* __restrict__ delta, float* __restrict__ nl2, uint16_t* __restrict__ dq, int64_t lddq, int S,
    int nh, int group, float scale_log2, float scale, RopeRows<uint16_t> rope) {
  constexpr int BM = 128, BN = 64, NS = HD / 16, ND = HD / 32, TILE = BN * 2 * HD;
  __shared__ __align__(16) char sk0[TILE], sk1[TILE], sv0[TILE], sv1[TILE];
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const XcdOrder ord = xcd_order();
  const int bh = ord.y, b = bh / nh, h = bh - b * nh, kvh = h / group;
  const int q0 = (gridDim.x - 1 - ord.rank) * BM;  // heaviest (latest) query blocks first
  const int qw = q0 + wave * 32, qi = qw + l32;
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  int a_off = lane_off_a<HD>(lane);
  int b0 = lane_off_b<HD>(lane, 0), b8 = lane_off_b<HD>(lane, 8);

  bf16x8 qf[NS], gf[NS];
  float nlse2 = 0.f, dl = 0.f;
  {
    const int64_t col = static_cast<int64_t>(h) * HD + 8 * hl;
    const uint16_t* qrow = q + (tok0 + qi) * ldq + col;
    const uint16_t* grow = dO + (tok0 + qi) * lddo + col;
    const uint16_t* orow = o + (tok0 + qi) * ldo + col;
    float part = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint4 gz = make_uint4(0, 0, 0, 0), oz = make_uint4(0, 0, 0, 0);
      qf[s] = as_bf16x8(gz);
      if (qi < S) {
        qf[s] = ld_frag(qrow + 16 * s);
        gz = *reinterpret_cast<const uint4*>(grow + 16 * s);
        oz = *reinterpret_cast<const uint4*>(orow + 16 * s);
      }
      gf[s] = as_bf16x8(gz);
      float gv[8], ov[8];
      Elem<uint16_t>::load8(reinterpret_cast<const uint16_t*>(&gz), gv);
      Elem<uint16_t>::load8(reinterpret_cast<const uint16_t*>(&oz), ov);
#pragma unroll
      for (int e = 0; e < 8; ++e) part = fmaf(gv[e], ov[e], part);
    }
    dl = xor32_sum(part);
    if (qi < S) {
      nlse2 = -lse[static_cast<int64_t>(bh) * S + qi] * kLog2e;
      if (hl == 0) {
        delta[static_cast<int64_t>(bh) * S + qi] = dl;
        nl2[static_cast<int64_t>(bh) * S + qi] = nlse2;
      }
    }
  }
  f32x16 dqacc[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) dqacc[dt] = zero16();

  const int kend = min(S, q0 + BM);
  const int nkb = (kend + BN - 1) / BN;
  const uint16_t* kb_ptr = k + tok0 * ldk + static_cast<int64_t>(kvh) * HD;
  const uint16_t* vb_ptr = v + tok0 * ldv + static_cast<int64_t>(kvh) * HD;
  kv_block_loop<BN, HD, false, 4>(kb_ptr, ldk, vb_ptr, ldv, nkb, S, sk0, sk1, sv0, sv1, wave, lane,
                        [&](int kb, const char* K, const char* V) __attribute__((always_inline)) {
                          refresh_offsets(a_off, b0, b8);
                          const int k0 = kb * BN;
                          if (k0 <= qw + 31)
                            dq_block<HD>(K, V, qf, gf, dqacc, nlse2, dl, a_off, b0, b8, k0, qw, qi, hl, S,
                                         scale_log2);
                        },
                        [] {});
  if (qi < S) store_grad_row<HD>(dq + (tok0 + qi) * lddq + static_cast<int64_t>(h) * HD, dqacc, scale, hl, rope, tok0, qi);
}

// Load stage of the dK/dV kernels: the Q and dO tiles, -lse*log2(e) and delta of one
// (query tile, query head) item of the loop, loaded straight into an LDS
// stage.  Items run from the last query tile down to the key block's first
// (qt0), and over the group's query heads within a tile: all blocks of one kv
// head start at the same tile and move down together, so a tile loaded by one
// block is found in L2 by the others.  q, dO, nl2, delta point at the group's
// first query head; nl2/delta rows are [head][S].  The tiles go through
// TileDma; the last wave loads -lse*log2(e) and delta of 64 rows from the
// tile's first (sl and sd hold 64 floats; rows from BQ on are unused).  Rows
// past S re-read row S - 1: the kernels mask their weights to zero.  No
// registers hold the tiles; the caller waits for its own loads (vmcnt) before
// the barrier that hands the stage to the other waves.
template <int HD, int BQ, int NT>
struct QTileDma {
  int qt = 0, hh = 0;  // the item to fetch next
  TileDma<BQ, HD, NT / 64> tq, tg;  // per-lane load offsets of the Q and dO tiles
  __device__ __forceinline__ void start(int qt_end, int64_t ldq, int64_t lddo, int wave, int lane) {
    qt = qt_end - 1;
    hh = 0;
    tq.init(ldq, wave, lane);
    tg.init(lddo, wave, lane);
  }
  __device__ __forceinline__ void advance(int group) {
    if (++hh == group) {
      hh = 0;
      --qt;
    }
  }
  __device__ __forceinline__ void fetch(const uint16_t* q, int64_t ldq, const uint16_t* dO,
                                        int64_t lddo, const float* nl2, const float* delta,
                                        int S, int qt0, int group, char* sq, char* sg, float* sl,
                                        float* sd, int wave, int lane) {
    typedef __attribute__((address_space(1))) const void* gptr;
    typedef __attribute__((address_space(3))) void* lptr;
    constexpr int NW = NT / 64;
    static_assert(BQ <= 64, "one lse/delta load covers the tile's rows");
    const int qs = max(qt, qt0) * BQ;
    const int64_t hcol = static_cast<int64_t>(hh) * HD;
    tq.load(q + hcol, ldq, qs, S - 1, sq, wave, lane);
    tg.load(dO + hcol, lddo, qs, S - 1, sg, wave, lane);
    if (wave == NW - 1) {
      const int64_t row = static_cast<int64_t>(hh) * S + min(qs + lane, S - 1);
      __builtin_amdgcn_global_load_lds((gptr)(nl2 + row), (lptr)sl, 4, 0, 0);
      __builtin_amdgcn_global_load_lds((gptr)(delta + row), (lptr)sd, 4, 0, 0);
    }
    advance(group);
  }
};

// ------------------------------------------ backward: dK, dV (bf16), fused roles
// Used for head_dim <= 64.  Block = 8 waves for one (batch, kv head) and two
// key blocks of 128 keys, j and nkb-1-j, taken one after the other (causal
// work per key block grows with the number of later queries, so every block
// carries the same work).  Within a key block, wave w holds K and V of keys
// 32*(w%4)..+31 in registers, and each 64-query tile is split between the two
// halves of the block: waves 0-3 take its queries 0-31, waves 4-7 queries
// 32-63.  So all 8 waves (two per SIMD) are busy in every iteration, and every
// block runs the same number of iterations.  The loop runs over the group's
// query heads and 64-query tiles (double-buffered in LDS, loaded straight
// into it):
//   S = Q K^T, P = exp(S - lse), dP = dO V^T, dS = P (dP - delta),
//   dV^T += dO^T P,  dK^T += Q^T dS,  dK = scale * dK.
// At the end of a key block the halves' partial dK and dV are exchanged
// through LDS and summed in a fixed order (half 0 + half 1): half 0 stores dK,
// half 1 stores dV.  Each kv head's gradient is complete inside one block: no
// atomics.
template <int HD>
struct DkdvFusedTiles {
  static constexpr int BQ = 64;
  static constexpr int NWH = 4;  // waves per query half (32 keys each)
  static constexpr int NT = 2 * NWH * 64;
};


// One wave's share of a query tile in the dK/dV kernel: the 32 queries at
// row hrow of the LDS tiles Q and dO (first query qh) against the wave's 32
// keys (first key kw, this lane's key ki), accumulated into dK^T and dV^T.
// The lane offsets a_off, b0, b8 already include row hrow.
template <int HD>
__device__ __forceinline__ void dkdv_tile(const char* Q, const char* G, const float* sl, const float* sd,
                                          const bf16x8 (&kf)[HD / 16], const bf16x8 (&vf)[HD / 16],
                                          f32x16 (&dkacc)[HD / 32], f32x16 (&dvacc)[HD / 32], int a_off,
                                          int b0, int b8, int hrow, int qh, int kw, int ki, int S,
                                          float scale_log2, int hl) {
  constexpr int NS = HD / 16, ND = HD / 32;
  const bool need_mask = (qh < kw + 31) || (qh + 32 > S) || (kw + 32 > S);
  f32x16 x = zero16(), y = zero16();  // S, dP (rows = queries, column = key ki)
  // Scheduling strategy 0 interleaves the LDS fragment reads with the MFMAs.
  __builtin_amdgcn_iglp_opt(0);
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    x = mfma(lds_frag<HD>(Q, a_off, 0, s), kf[s], x);
    y = mfma(lds_frag<HD>(G, a_off, 0, s), vf[s], y);
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 L4 = *reinterpret_cast<const float4*>(&sl[hrow + 8 * g + 4 * hl]);
    const float4 D4 = *reinterpret_cast<const float4*>(&sd[hrow + 8 * g + 4 * hl]);
    const float Lv[4] = {L4.x, L4.y, L4.z, L4.w};  // -lse * log2(e)
    const float Dv[4] = {D4.x, D4.y, D4.z, D4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 4 * g + e;
      const float p = fast_exp2(fmaf(x[j], scale_log2, Lv[e]));
      x[j] = p;                   // P
      y[j] = p * (y[j] - Dv[e]);  // dS
    }
  }
  if (need_mask) {
    // query qa = qh + acc_row(j, hl) is dead for this lane's key ki when
    // qa < ki, qa >= S or ki >= S: its compile-time part acc_row(j, 0) lies
    // outside [lo, hi) (an empty range when ki >= S).
    const int lo = ki - qh - 4 * hl, hi = ki < S ? S - qh - 4 * hl : lo;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const bool dead = static_cast<int>(acc_row(j, 0) < lo) | static_cast<int>(acc_row(j, 0) >= hi);
      x[j] = dead ? 0.f : x[j];
      y[j] = dead ? 0.f : y[j];
    }
  }
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    const bf16x8 pf = pack_frag(x, 8 * s2);
    const bf16x8 df = pack_frag(y, 8 * s2);
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      dvacc[dt] = mfma(lds_frag_tr<HD>(G, b0, b8, 16 * s2, dt), pf, dvacc[dt]);
      dkacc[dt] = mfma(lds_frag_tr<HD>(Q, b0, b8, 16 * s2, dt), df, dkacc[dt]);
    }
  }
}

template <int HD>
__global__ __launch_bounds__(DkdvFusedTiles<HD>::NT) __attribute__((amdgpu_waves_per_eu(2))) void k_attn_bwd_dkdv_fused(
    const uint16_t* __restrict__ q, int64_t ldq, const uint16_t* __restrict__ k, int64_t ldk,
    const uint16_t* __restrict__ v, int64_t ldv, const uint16_t* __restrict__ dO, int64_t lddo,
    const float* __restrict__ nl2, const float* __restrict__ delta, uint16_t* __restrict__ dk,
    int64_t lddk, uint16_t* __restrict__ dv, int64_t lddv, int S, int nh, int nkv, int group,
    float scale_log2, float scale, RopeRows<uint16_t> rope) {
  constexpr int NWH = DkdvFusedTiles<HD>::NWH, NT = DkdvFusedTiles<HD>::NT;
  constexpr int BKN = NWH * 32, BQ = DkdvFusedTiles<HD>::BQ, NS = HD / 16, ND = HD / 32;
  constexpr int TILE = BQ * 2 * HD;
  static_assert(BQ == 64 && BKN % BQ == 0, "two 32-query halves per tile; key blocks align with tiles");
  // Two LDS stages as separate arrays: the loop is unrolled by two, so every
  // access names its stage statically and the compiler can tell that the
  // direct-to-LDS loads into one stage do not alias the reads of the other.
  // One struct fixes the layout: the tiles the loop reads first, below 64 KB,
  // so that their base is a read's immediate offset (placed after the 64 KB
  // exchange buffer, every tile read added its base in a VGPR).
  // Two items per stage (IPB): the barrier that ends a stage comes once per
  // two items, halving the waits for the slowest wave.
  struct Lds {
    char sq0a[TILE], sq0b[TILE], sq1a[TILE], sq1b[TILE];
    char sg0a[TILE], sg0b[TILE], sg1a[TILE], sg1b[TILE];
    float sl0a[BQ], sl0b[BQ], sl1a[BQ], sl1b[BQ];  // -lse*log2(e)
    float sd0a[BQ], sd0b[BQ], sd1a[BQ], sd1b[BQ];  // delta
    float xchg[2][NWH][ND * 16][64];               // [0]: dV of half 0, [1]: dK of half 1
  };
  static_assert(8 * TILE <= 65536, "every tile read's base fits a ds_read immediate");
  __shared__ __align__(16) Lds lds;
  auto& xchg = lds.xchg;
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const int half = wave / NWH, wq = wave % NWH;
  const XcdOrder ord = xcd_order();
  const int bk = ord.y, b = bk / nkv, kvh = bk - b * nkv;
  const int nkb = (S + BKN - 1) / BKN;
  const int jlo = ord.rank, jhi = nkb - 1 - ord.rank;
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  const int hrow = 32 * half;  // this wave's first query row within a tile
  // The LDS read offsets include the wave's first row (its byte offset lies
  // above the bits the swizzle XORs touch, so it commutes with them): the
  // tile reads are then a lane offset plus an immediate, with no address
  // additions in the loop (32 per query tile otherwise).
  int a_off = lane_off_a<HD>(lane) + hrow * 2 * HD;
  int b0 = lane_off_b<HD>(lane, 0) + hrow * 2 * HD, b8 = lane_off_b<HD>(lane, 8) + hrow * 2 * HD;
  const int64_t h0 = static_cast<int64_t>(kvh) * group;
  const uint16_t* qg = q + tok0 * ldq + h0 * HD;
  const uint16_t* gg = dO + tok0 * lddo + h0 * HD;
  const float* lg = nl2 + (static_cast<int64_t>(b) * nh + h0) * S;
  const float* dg = delta + (static_cast<int64_t>(b) * nh + h0) * S;
  const int qt_end = (S + BQ - 1) / BQ;

  for (int ph = 0; ph < 2; ++ph) {
    if (ph == 1 && jhi <= jlo) break;  // block-uniform: the middle key block of an odd count
    const int jb = ph == 0 ? jlo : jhi;
    const int kw = jb * BKN + wq * 32, ki = kw + l32;
    bf16x8 kf[NS], vf[NS];
    {
      const bool ok = ki < S;
      const uint16_t* krow = k + (tok0 + ki) * ldk + static_cast<int64_t>(kvh) * HD + 8 * hl;
      const uint16_t* vrow = v + (tok0 + ki) * ldv + static_cast<int64_t>(kvh) * HD + 8 * hl;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        kf[s] = ok ? ld_frag(krow + 16 * s) : as_bf16x8(make_uint4(0, 0, 0, 0));
        vf[s] = ok ? ld_frag(vrow + 16 * s) : as_bf16x8(make_uint4(0, 0, 0, 0));
      }
    }
    f32x16 dkacc[ND], dvacc[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      dkacc[dt] = zero16();
      dvacc[dt] = zero16();
    }

    // Iteration space: (query tiles from the key block's first key, last tile
    // first) x (query heads of the group), n_it >= 1 items.  Item it + 1 is
    // loaded straight into the other LDS stage while item it is multiplied;
    // each wave waits for its own loads before the barrier that ends the item.
    const int qt0 = (jb * BKN) / BQ;
    const int n_it = group * (qt_end - qt0);
    QTileDma<HD, BQ, NT> pre;
    pre.start(qt_end, ldq, lddo, wave, lane);
    pre.fetch(qg, ldq, gg, lddo, lg, dg, S, qt0, group, lds.sq0a, lds.sg0a, lds.sl0a, lds.sd0a, wave, lane);
    if (n_it > 1)
      pre.fetch(qg, ldq, gg, lddo, lg, dg, S, qt0, group, lds.sq0b, lds.sg0b, lds.sl0b, lds.sd0b, wave, lane);
    wait_loads();
    __syncthreads();
    int cqt = qt_end - 1, chh = 0;  // query tile and head of the current item
    // Item IT from (QC, GC, LC, DC), and item IT + 2 into (QN, GN, LN, DN).
#define FH_DKDV_ITEM(IT, QC, GC, LC, DC, QN, GN, LN, DN)                                          \
  {                                                                                               \
    refresh_offsets(a_off, b0, b8);                                                               \
    if ((IT) + 2 < n_it)                                                                          \
      pre.fetch(qg, ldq, gg, lddo, lg, dg, S, qt0, group, QN, GN, LN, DN, wave, lane);            \
    const int qh = cqt * BQ + hrow; /* first query of this wave's half */                         \
    if ((IT) < n_it && qh + 31 >= kw) /* some query of the half reaches this wave's keys */      \
      dkdv_tile<HD>(QC, GC, LC, DC, kf, vf, dkacc, dvacc, a_off, b0, b8, hrow, qh, kw, ki, S,      \
                    scale_log2, hl);                                                              \
    if (++chh == group) {                                                                         \
      chh = 0;                                                                                    \
      --cqt;                                                                                      \
    }                                                                                             \
  }
    // Stage 0 holds items it, it + 1 while items it + 2, it + 3 are loaded
    // into stage 1; each wave waits for its own loads before the barrier that
    // ends the pair.
    for (int it = 0; it < n_it; it += 4) {
      FH_DKDV_ITEM(it, lds.sq0a, lds.sg0a, lds.sl0a, lds.sd0a, lds.sq1a, lds.sg1a, lds.sl1a, lds.sd1a)
      FH_DKDV_ITEM(it + 1, lds.sq0b, lds.sg0b, lds.sl0b, lds.sd0b, lds.sq1b, lds.sg1b, lds.sl1b, lds.sd1b)
      wait_loads();
      __syncthreads();
      FH_DKDV_ITEM(it + 2, lds.sq1a, lds.sg1a, lds.sl1a, lds.sd1a, lds.sq0a, lds.sg0a, lds.sl0a, lds.sd0a)
      FH_DKDV_ITEM(it + 3, lds.sq1b, lds.sg1b, lds.sl1b, lds.sd1b, lds.sq0b, lds.sg0b, lds.sl0b, lds.sd0b)
      wait_loads();
      __syncthreads();
    }
#undef FH_DKDV_ITEM

    // Sum the halves: half 0 hands over its dV, half 1 its dK.
    float(*mine)[64] = xchg[half][wq];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int j = 0; j < 16; ++j) mine[dt * 16 + j][lane] = half == 0 ? dvacc[dt][j] : dkacc[dt][j];
    __syncthreads();
    const float(*other)[64] = xchg[half ^ 1][wq];
    if (half == 0) {
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) dkacc[dt][j] = dkacc[dt][j] + other[dt * 16 + j][lane];
      if (ki < S) store_grad_row<HD>(dk + (tok0 + ki) * lddk + static_cast<int64_t>(kvh) * HD, dkacc, scale, hl, rope, tok0, ki);
    } else {
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) dvacc[dt][j] = other[dt * 16 + j][lane] + dvacc[dt][j];
      if (ki < S) store_rows_T<HD>(dv + (tok0 + ki) * lddv + static_cast<int64_t>(kvh) * HD, dvacc, 1.f, hl);
    }
  }
}

// ------------------------------------------ backward: dK, dV (bf16), split roles
// Used for head_dim 128.  Block = one key block of 32*NKS keys of one (batch,
// kv head), 2*NKS waves.  Each 32-key sub-tile is shared by two waves with
// different roles, so that no wave carries both the dK and the dV accumulators
// (that would need ~300 registers at head_dim 128, i.e. one wave per SIMD):
//   wave A (waves 0..NKS-1):    holds K;  S = Q K^T, P = exp(S - lse) -> LDS
//                               (fp32), dV^T += dO^T P
//   wave B (waves NKS..2NKS-1): holds V;  dP = dO V^T, dS = P (dP - delta) with
//                               P read from LDS, dK^T += Q^T dS, dK = scale * dK
// Every query tile runs in two phases separated by a barrier: phase 1 forms S
// (A) and dP (B), phase 2 the two accumulating products; both roles issue the
// same number of MFMAs in each phase.  The loop runs over the GQA group's query
// heads and the BQ-query tiles at or after the block's first key (Q, dO, lse
// and delta double-buffered in LDS, loaded straight into it), so each kv
// head's gradient is complete inside one block: no atomics.  Blocks are
// numbered heaviest (earliest keys, most causal work) first.
template <int HD>
struct DkdvTiles {
  static constexpr int NKS = 2;  // 32-key sub-tiles per block
  static constexpr int BQ = 32;  // queries per tile
  static constexpr int NT = 2 * NKS * 64;
};

template <int HD>
__global__ __launch_bounds__(DkdvTiles<HD>::NT) __attribute__((amdgpu_waves_per_eu(2))) void k_attn_bwd_dkdv(
    const uint16_t* __restrict__ q, int64_t ldq, const uint16_t* __restrict__ k, int64_t ldk,
    const uint16_t* __restrict__ v, int64_t ldv, const uint16_t* __restrict__ dO, int64_t lddo,
    const float* __restrict__ nl2, const float* __restrict__ delta, uint16_t* __restrict__ dk,
    int64_t lddk, uint16_t* __restrict__ dv, int64_t lddv, int S, int nh, int nkv, int group,
    float scale_log2, float scale, RopeRows<uint16_t> rope) {
  constexpr int NKS = DkdvTiles<HD>::NKS, NT = DkdvTiles<HD>::NT, BQ = DkdvTiles<HD>::BQ;
  constexpr int BKN = NKS * 32, NS = HD / 16, ND = HD / 32, NQT = BQ / 32, TILE = BQ * 2 * HD;
  // Two LDS stages as separate arrays (the loop below is unrolled by two),
  // each the Q tile followed by the dO tile: a role picks its tile by offset
  // within the stage's array, so the compiler still knows which array each
  // read touches (with a pointer chosen between two arrays it would wait for
  // every load in flight first).  lse and delta rows are loaded 64 at a time;
  // rows from BQ on are unused.
  __shared__ __align__(16) char st0[2 * TILE], st1[2 * TILE];
  __shared__ __align__(16) float sl0[64], sl1[64], sd0[64], sd1[64];  // -lse*log2(e) and delta
  __shared__ __align__(16) float sp[NKS][NQT][16 * 64];  // P of each sub-tile, [j/4][lane][4]
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar) index
  const bool role_a = wave < NKS;
  const int sub = role_a ? wave : wave - NKS;
  const XcdOrder ord = xcd_order();
  const int bk = ord.y, b = bk / nkv, kvh = bk - b * nkv;
  const int kb0 = ord.rank * BKN;  // heaviest (earliest keys) first
  const int kw = kb0 + sub * 32, ki = kw + l32;
  const int64_t tok0 = static_cast<int64_t>(b) * S;
  int a_off = lane_off_a<HD>(lane);
  int b0 = lane_off_b<HD>(lane, 0), b8 = lane_off_b<HD>(lane, 8);

  bf16x8 kv[NS];  // K (role A) or V (role B) of this lane's key
  {
    const uint16_t* src = role_a ? k + (tok0 + ki) * ldk : v + (tok0 + ki) * ldv;
    src += static_cast<int64_t>(kvh) * HD + 8 * hl;
#pragma unroll
    for (int s = 0; s < NS; ++s) kv[s] = ki < S ? ld_frag(src + 16 * s) : as_bf16x8(make_uint4(0, 0, 0, 0));
  }
  f32x16 acc[ND];  // dV^T (role A) or dK^T (role B)
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) acc[dt] = zero16();

  // iteration space: (query tiles from the block's first key, last first) x (query heads of the group)
  const int qt0 = kb0 / BQ, qt_end = (S + BQ - 1) / BQ;
  const int n_it = group * (qt_end - qt0);
  const int64_t h0 = static_cast<int64_t>(kvh) * group;
  const uint16_t* qg = q + tok0 * ldq + h0 * HD;
  const uint16_t* gg = dO + tok0 * lddo + h0 * HD;
  const float* lg = nl2 + (static_cast<int64_t>(b) * nh + h0) * S;
  const float* dg = delta + (static_cast<int64_t>(b) * nh + h0) * S;
  QTileDma<HD, BQ, NT> pre;
  pre.start(qt_end, ldq, lddo, wave, lane);
  if (n_it > 0) pre.fetch(qg, ldq, gg, lddo, lg, dg, S, qt0, group, st0, st0 + TILE, sl0, sd0, wave, lane);
  wait_loads();
  __syncthreads();
  int cqt = qt_end - 1, chh = 0;  // query tile and head of the current item
  const int xoff = role_a ? 0 : TILE;  // phase 1 reads Q (A) or dO (B), phase 2 the other
  // Item it from stage (T, L, D) while item it + 1 is loaded into stage (TN, LN, DN).
  auto step = [&](int it, const char* T, const float* L, const float* D, char* TN, float* LN, float* DN)
                  __attribute__((always_inline)) {
    refresh_offsets(a_off, b0, b8);
    if (it + 1 < n_it) pre.fetch(qg, ldq, gg, lddo, lg, dg, S, qt0, group, TN, TN + TILE, LN, DN, wave, lane);
    const int q0 = cqt * BQ;
    // some query of the tile reaches this sub-tile's keys (same answer for both roles)
    const bool active = it < n_it && kw < S && q0 + BQ - 1 >= kw;
    const bool need_mask = (q0 < kw + 31) || (q0 + BQ > S) || (kw + 32 > S);
    f32x16 x[NQT];  // S then P (role A) / dP then dS (role B), rows = queries, column = key ki
    // phase 1: S = Q K^T, P = exp(S - lse) -> LDS (A) or dP = dO V^T (B)
    if (active) {
      const char* X = T + xoff;
#pragma unroll
      for (int u = 0; u < NQT; ++u) {
        x[u] = zero16();
#pragma unroll
        for (int s = 0; s < NS; ++s) x[u] = mfma(lds_frag<HD>(X, a_off, 32 * u, s), kv[s], x[u]);
      }
      if (role_a) {
#pragma unroll
        for (int u = 0; u < NQT; ++u) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 L4 = *reinterpret_cast<const float4*>(&L[32 * u + 8 * g + 4 * hl]);
            const float Lv[4] = {L4.x, L4.y, L4.z, L4.w};  // -lse * log2(e)
#pragma unroll
            for (int e = 0; e < 4; ++e) x[u][4 * g + e] = fast_exp2(fmaf(x[u][4 * g + e], scale_log2, Lv[e]));
          }
          if (need_mask) {  // also zeroes the rows past S (their Q/dO rows repeat row S - 1)
            // query qa = q0 + 32u + acc_row(j, hl) is dead when qa < ki, qa >= S
            // or ki >= S: acc_row(j, 0) outside [lo, hi) (empty when ki >= S).
            const int lo = ki - q0 - 32 * u - 4 * hl, hi = ki < S ? S - q0 - 32 * u - 4 * hl : lo;
#pragma unroll
            for (int j = 0; j < 16; ++j)
              x[u][j] = (static_cast<int>(acc_row(j, 0) < lo) | static_cast<int>(acc_row(j, 0) >= hi)) ? 0.f : x[u][j];
          }
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *reinterpret_cast<float4*>(&sp[sub][u][(g * 64 + lane) * 4]) =
                make_float4(x[u][4 * g], x[u][4 * g + 1], x[u][4 * g + 2], x[u][4 * g + 3]);
        }
      }
    }
    lds_barrier();  // P is in LDS; the loads into the other stage may still be in flight
    // phase 2: dV^T += dO^T P (A) or dS = P (dP - delta), dK^T += Q^T dS (B)
    if (active) {
      if (!role_a) {
#pragma unroll
        for (int u = 0; u < NQT; ++u)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 D4 = *reinterpret_cast<const float4*>(&D[32 * u + 8 * g + 4 * hl]);
            const float4 P4 = *reinterpret_cast<const float4*>(&sp[sub][u][(g * 64 + lane) * 4]);
            const float Dv[4] = {D4.x, D4.y, D4.z, D4.w};
            const float Pv[4] = {P4.x, P4.y, P4.z, P4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) x[u][4 * g + e] = Pv[e] * (x[u][4 * g + e] - Dv[e]);
          }
      }
      const char* Y = T + (TILE - xoff);
#pragma unroll
      for (int u = 0; u < NQT; ++u)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const bf16x8 f = pack_frag(x[u], 8 * s2);
#pragma unroll
          for (int dt = 0; dt < ND; ++dt)
            acc[dt] = mfma(lds_frag_tr<HD>(Y, b0, b8, 32 * u + 16 * s2, dt), f, acc[dt]);
        }
    }
    if (++chh == group) {
      chh = 0;
      --cqt;
    }
    wait_loads();
    __syncthreads();
  };
  for (int it = 0; it < n_it; it += 2) {
    step(it, st0, sl0, sd0, st1, sl1, sd1);
    step(it + 1, st1, sl1, sd1, st0, sl0, sd0);
  }
  if (ki < S) {
    if (role_a)
      store_rows_T<HD>(dv + (tok0 + ki) * lddv + static_cast<int64_t>(kvh) * HD, acc, 1.f, hl);
    else
      store_grad_row<HD>(dk + (tok0 + ki) * lddk + static_cast<int64_t>(kvh) * HD, acc, scale, hl, rope, tok0, ki);
  }
}

// --------------------------------------------------------- fp32 reference-precision kernels
// Plain fp32 FMA kernels (one thread per output row) for fp32 models; the same
// algorithm (online softmax forward with lse, delta-based backward) as above.

// out[d] = acc[d] * mul, followed by the RoPE backward of the row when
// rope.cos is set (the fp32 counterpart of store_grad_row).
template <int HD>
__device__ __forceinline__ void store_row_f32(float* out, const float (&acc)[HD], float mul,
                                              const RopeRows<float>& rope, int64_t tok0, int pos) {
  if (!rope.cos) {
    for (int d = 0; d < HD; ++d) out[d] = acc[d] * mul;
    return;
  }
  const int64_t r = rope.row(tok0, pos) * HD;
  const float* cs = rope.cos + r;
  const float* sn = rope.sin + r;
  for (int d = 0; d < HD / 2; ++d) {
    float o0, o1;
    rope_pair<float, true>(acc[d] * mul, acc[d + HD / 2] * mul, cs[d], cs[d + HD / 2], sn[d], sn[d + HD / 2],
                           o0, o1);
    out[d] = o0;
    out[d + HD / 2] = o1;
  }
}
template <int HD>
__global__ __launch_bounds__(128) void k_attn_fwd_f32(
    const float* q, int64_t ldq, const float* __restrict__ k, int64_t ldk,
    const float* __restrict__ v, int64_t ldv, float* __restrict__ o, int64_t ldo,
    float* __restrict__ lse, int S, int nh, int group, float scale, int64_t rows, RopeRows<float> rope,
    float* qout, int64_t ldqo) {  // q and qout may alias (in-place rotated q)
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows) return;  // rows = B*nh*S, idx = (b*nh + h)*S + s
  const int s = static_cast<int>(idx % S);
  const int64_t bh = idx / S;
  const int h = static_cast<int>(bh % nh);
  const int64_t b = bh / nh;
  const int kvh = h / group;
  const float* qr = q + (b * S + s) * ldq + static_cast<int64_t>(h) * HD;
  float qv[HD], acc[HD];
  for (int d = 0; d < HD; ++d) { qv[d] = qr[d]; acc[d] = 0.f; }
  if (rope.cos) {  // q rotated on load (RoPE forward), optionally written back
    const int64_t r = rope.row(b * S, s) * HD;
    float* qo = qout ? qout + (b * S + s) * ldqo + static_cast<int64_t>(h) * HD : nullptr;
    for (int d = 0; d < HD / 2; ++d) {
      float o0, o1;
      rope_pair<float, false>(qv[d], qv[d + HD / 2], rope.cos[r + d], rope.cos[r + d + HD / 2], rope.sin[r + d],
                              rope.sin[r + d + HD / 2], o0, o1);
      qv[d] = o0;
      qv[d + HD / 2] = o1;
      if (qo) {
        qo[d] = o0;
        qo[d + HD / 2] = o1;
      }
    }
  }
  float m = -INFINITY, l = 0.f;
  for (int j = 0; j <= s; ++j) {
    const float* kr = k + (b * S + j) * ldk + static_cast<int64_t>(kvh) * HD;
    const float* vr = v + (b * S + j) * ldv + static_cast<int64_t>(kvh) * HD;
    float x = 0.f;
    for (int d = 0; d < HD; ++d) x = fmaf(qv[d], kr[d], x);
    x *= scale;
    const float mn = fmaxf(m, x);
    const float a = expf(m - mn), p = expf(x - mn);
    l = l * a + p;
    for (int d = 0; d < HD; ++d) acc[d] = acc[d] * a + p * vr[d];
    m = mn;
  }
  float* orow = o + (b * S + s) * ldo + static_cast<int64_t>(h) * HD;
  for (int d = 0; d < HD; ++d) orow[d] = acc[d] / l;
  if (lse != nullptr) lse[idx] = m + logf(l);
}

template <int HD>
__global__ __launch_bounds__(128) void k_attn_bwd_dq_f32(
    const float* __restrict__ q, int64_t ldq, const float* __restrict__ k, int64_t ldk,
    const float* __restrict__ v, int64_t ldv, const float* __restrict__ dO, int64_t lddo,
    const float* __restrict__ lse, const float* __restrict__ delta, float* __restrict__ dq,
    int64_t lddq, int S, int nh, int group, float scale, int64_t rows, RopeRows<float> rope) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows) return;
  const int s = static_cast<int>(idx % S);
  const int64_t bh = idx / S;
  const int h = static_cast<int>(bh % nh);
  const int64_t b = bh / nh;
  const int kvh = h / group;
  const float* qr = q + (b * S + s) * ldq + static_cast<int64_t>(h) * HD;
  const float* gr = dO + (b * S + s) * lddo + static_cast<int64_t>(h) * HD;
  float qv[HD], gv[HD], acc[HD];
  for (int d = 0; d < HD; ++d) { qv[d] = qr[d]; gv[d] = gr[d]; acc[d] = 0.f; }
  const float L = lse[idx], D = delta[idx];
  for (int j = 0; j <= s; ++j) {
    const float* kr = k + (b * S + j) * ldk + static_cast<int64_t>(kvh) * HD;
    const float* vr = v + (b * S + j) * ldv + static_cast<int64_t>(kvh) * HD;
    float x = 0.f, dp = 0.f;
    for (int d = 0; d < HD; ++d) {
      x = fmaf(qv[d], kr[d], x);
      dp = fmaf(gv[d], vr[d], dp);
    }
    const float ds = expf(x * scale - L) * (dp - D);
    for (int d = 0; d < HD; ++d) acc[d] = fmaf(ds, kr[d], acc[d]);
  }
  float* out = dq + (b * S + s) * lddq + static_cast<int64_t>(h) * HD;
  store_row_f32<HD>(out, acc, scale, rope, b * S, s);
}

template <int HD>
__global__ __launch_bounds__(128) void k_attn_bwd_dkdv_f32(
    const float* __restrict__ q, int64_t ldq, const float* __restrict__ k, int64_t ldk,
    const float* __restrict__ v, int64_t ldv, const float* __restrict__ dO, int64_t lddo,
    const float* __restrict__ lse, const float* __restrict__ delta, float* __restrict__ dk,
    int64_t lddk, float* __restrict__ dv, int64_t lddv, int S, int nh, int nkv, int group,
    float scale, int64_t rows, RopeRows<float> rope) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows) return;  // rows = B*nkv*S, idx = (b*nkv + kvh)*S + j
  const int j = static_cast<int>(idx % S);
  const int64_t bk = idx / S;
  const int kvh = static_cast<int>(bk % nkv);
  const int64_t b = bk / nkv;
  const float* kr = k + (b * S + j) * ldk + static_cast<int64_t>(kvh) * HD;
  const float* vr = v + (b * S + j) * ldv + static_cast<int64_t>(kvh) * HD;
  float kv[HD], vv[HD], ak[HD], av[HD];
  for (int d = 0; d < HD; ++d) { kv[d] = kr[d]; vv[d] = vr[d]; ak[d] = 0.f; av[d] = 0.f; }
  for (int hh = 0; hh < group; ++hh) {
    const int h = kvh * group + hh;
    const int64_t row = (b * nh + h) * S;
    for (int s = j; s < S; ++s) {
      const float* qr = q + (b * S + s) * ldq + static_cast<int64_t>(h) * HD;
      const float* gr = dO + (b * S + s) * lddo + static_cast<int64_t>(h) * HD;
      float x = 0.f, dp = 0.f;
      for (int d = 0; d < HD; ++d) {
        x = fmaf(qr[d], kv[d], x);
        dp = fmaf(gr[d], vv[d], dp);
      }
      const float p = expf(x * scale - lse[row + s]);
      const float ds = p * (dp - delta[row + s]);
      for (int d = 0; d < HD; ++d) {
        av[d] = fmaf(p, gr[d], av[d]);
        ak[d] = fmaf(ds, qr[d], ak[d]);
      }
    }
  }
  float* ok = dk + (b * S + j) * lddk + static_cast<int64_t>(kvh) * HD;
  float* ov = dv + (b * S + j) * lddv + static_cast<int64_t>(kvh) * HD;
  for (int d = 0; d < HD; ++d) ov[d] = av[d];
  store_row_f32<HD>(ok, ak, scale, rope, b * S, j);
}

// ------------------------------------------------------------------- host
struct Dims {
  int64_t B, S, nh, nkv, hd;
};

int check_dims(fh_dtype dt, const Dims& d) {
  FH_REQUIRE(dt == FH_BF16 || dt == FH_F32, "attention: dtype must be FH_BF16 or FH_F32");
  FH_REQUIRE(d.B >= 0 && d.S >= 0, "attention: negative batch/seq_len");
  FH_REQUIRE(d.nh > 0 && d.nkv > 0 && d.nh % d.nkv == 0,
             "attention: n_heads must be a positive multiple of n_kv_heads");
  FH_REQUIRE(d.hd == 32 || d.hd == 64 || d.hd == 128, "attention: head_dim must be 32, 64 or 128");
  FH_REQUIRE(d.S <= (int64_t(1) << 30) && d.B * d.nh <= 65535 && d.B * d.nkv <= 65535,
             "attention: grid too large");
  return FH_OK;
}

int check_ld(int64_t ld, int64_t heads, int64_t hd, const char* what) {
  // < 2^24: the kernels' per-lane tile load offsets (up to 64 rows) are 32-bit
  if (ld < heads * hd || ld % 8 != 0 || ld >= (int64_t(1) << 24))
    return fail(FH_ERR_INVALID, std::string("attention: ") + what +
                                    " row stride must be >= heads*head_dim, a multiple of 8 and < 2^24");
  return FH_OK;
}

template <typename F>
int dispatch_hd(int64_t hd, F&& f) {
  if (hd == 32) return f(std::integral_constant<int, 32>{});
  if (hd == 64) return f(std::integral_constant<int, 64>{});
  return f(std::integral_constant<int, 128>{});
}

}  // namespace
}  // namespace fh

using namespace fh;

extern "C" size_t fh_attn_bwd_workspace_size(int64_t batch, int64_t seq_len, int64_t n_heads) {
  if (batch <= 0 || seq_len <= 0 || n_heads <= 0) return 0;
  return 2 * static_cast<size_t>(batch * seq_len * n_heads) * sizeof(float);
}

namespace {

// Rotary tables as passed to the *_rope entry points (cos == null: no rotation).
struct RopeArgs {
  const void* cos;
  const void* sin;
  int per_token;
};

int attn_fwd_impl(fh_dtype dt, const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                  int64_t ldv, void* o, int64_t ldo, float* lse, void* qout, int64_t ldqo, int64_t batch,
                  int64_t seq_len, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, float scale,
                  const RopeArgs& rp, hipStream_t stream) {
  const Dims d{batch, seq_len, n_heads, n_kv_heads, head_dim};
  if (int e = check_dims(dt, d)) return e;
  if (batch == 0 || seq_len == 0) return FH_OK;
  if (int e = check_ld(ldq, n_heads, head_dim, "q")) return e;
  if (int e = check_ld(ldk, n_kv_heads, head_dim, "k")) return e;
  if (int e = check_ld(ldv, n_kv_heads, head_dim, "v")) return e;
  if (int e = check_ld(ldo, n_heads, head_dim, "o")) return e;
  FH_REQUIRE(q && k && v && o, "attn_fwd: null pointer");
  FH_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o),
             "attn_fwd: pointers must be 16-byte aligned");
  if (qout) {
    if (int e = check_ld(ldqo, n_heads, head_dim, "q_out")) return e;
    FH_REQUIRE(aligned16(qout), "attn_fwd_rope: q_out must be 16-byte aligned");
    FH_REQUIRE(qout != q || ldqo == ldq, "attn_fwd_rope: q_out aliasing q must share its row stride");
  }
  const int S = static_cast<int>(seq_len), nh = static_cast<int>(n_heads);
  const int group = static_cast<int>(n_heads / n_kv_heads);
  if (dt == FH_BF16) {
    const RopeRows<uint16_t> rb{static_cast<const uint16_t*>(rp.cos), static_cast<const uint16_t*>(rp.sin),
                                rp.per_token};
    dispatch_hd(head_dim, [&](auto hdc) {
      constexpr int BM = 4 * 32 * FwdTiles<decltype(hdc)::value>::QT;
      const bool pair = group % 2 == 0 && (batch * n_heads / 2) % 8 == 0;
      const dim3 grid(static_cast<unsigned>((seq_len + BM - 1) / BM),
                      static_cast<unsigned>(batch * n_heads / (pair ? 2 : 1)));
      if (pair)
        hipLaunchKernelGGL((k_attn_fwd<hdc(), 2>), grid, dim3(512), 0, stream,
                           static_cast<const uint16_t*>(q), ldq, static_cast<const uint16_t*>(k), ldk,
                           static_cast<const uint16_t*>(v), ldv, static_cast<uint16_t*>(o), ldo, lse,
                           S, nh, group, scale * kLog2e, rb, static_cast<uint16_t*>(qout), ldqo);
      else
        hipLaunchKernelGGL((k_attn_fwd<hdc(), 1>), grid, dim3(256), 0, stream,
                           static_cast<const uint16_t*>(q), ldq, static_cast<const uint16_t*>(k), ldk,
                           static_cast<const uint16_t*>(v), ldv, static_cast<uint16_t*>(o), ldo, lse,
                           S, nh, group, scale * kLog2e, rb, static_cast<uint16_t*>(qout), ldqo);
      return 0;
    });
  } else {
    const RopeRows<float> rf{static_cast<const float*>(rp.cos), static_cast<const float*>(rp.sin), rp.per_token};
    const int64_t rows = batch * n_heads * seq_len;
    dispatch_hd(head_dim, [&](auto hdc) {
      hipLaunchKernelGGL((k_attn_fwd_f32<hdc()>), dim3(static_cast<unsigned>((rows + 127) / 128)),
                         dim3(128), 0, stream, static_cast<const float*>(q), ldq,
                         static_cast<const float*>(k), ldk, static_cast<const float*>(v), ldv,
                         static_cast<float*>(o), ldo, lse, S, nh, group, scale, rows, rf,
                         static_cast<float*>(qout), ldqo);
      return 0;
    });
  }
  return check_launch(rp.cos ? "fh_attn_fwd_rope" : "fh_attn_fwd");
}

}  // namespace

extern "C" int fh_attn_fwd(fh_dtype dt, const void* q, int64_t ldq, const void* k, int64_t ldk,
                           const void* v, int64_t ldv, void* o, int64_t ldo, float* lse,
                           int64_t batch, int64_t seq_len, int64_t n_heads, int64_t n_kv_heads,
                           int64_t head_dim, float scale, hipStream_t stream) {
  return attn_fwd_impl(dt, q, ldq, k, ldk, v, ldv, o, ldo, lse, nullptr, 0, batch, seq_len, n_heads, n_kv_heads,
                       head_dim, scale, RopeArgs{nullptr, nullptr, 0}, stream);
}

extern "C" int fh_attn_fwd_rope(fh_dtype dt, const void* q, int64_t ldq, const void* k, int64_t ldk,
                                const void* v, int64_t ldv, void* o, int64_t ldo, float* lse, void* q_out,
                                int64_t ldqo, int64_t batch, int64_t seq_len, int64_t n_heads,
                                int64_t n_kv_heads, int64_t head_dim, float scale, const void* cos,
                                const void* sin, int cos_per_token, hipStream_t stream) {
  FH_REQUIRE(cos && sin, "attn_fwd_rope: null cos/sin");
  FH_REQUIRE(aligned16(cos) && aligned16(sin), "attn_fwd_rope: cos/sin must be 16-byte aligned");
  return attn_fwd_impl(dt, q, ldq, k, ldk, v, ldv, o, ldo, lse, q_out, ldqo, batch, seq_len, n_heads,
                       n_kv_heads, head_dim, scale, RopeArgs{cos, sin, cos_per_token ? 1 : 0}, stream);
}

namespace {

int attn_bwd_impl(fh_dtype dt, const void* q, int64_t ldq, const void* k, int64_t ldk, const void* v,
                  int64_t ldv, const void* o, int64_t ldo, const void* dout, int64_t lddo, const float* lse,
                  void* dq, int64_t lddq, void* dk, int64_t lddk, void* dv, int64_t lddv, void* workspace,
                  int64_t batch, int64_t seq_len, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                  float scale, const RopeArgs& rp, hipStream_t stream) {
  const Dims d{batch, seq_len, n_heads, n_kv_heads, head_dim};
  if (int e = check_dims(dt, d)) return e;
  if (batch == 0 || seq_len == 0) return FH_OK;
  struct LdCheck {
    int64_t ld, heads;
    const char* what;
  };
  const LdCheck lds[] = {{ldq, n_heads, "q"},   {ldk, n_kv_heads, "k"}, {ldv, n_kv_heads, "v"},
                         {ldo, n_heads, "o"},   {lddo, n_heads, "dout"}, {lddq, n_heads, "dq"},
                         {lddk, n_kv_heads, "dk"}, {lddv, n_kv_heads, "dv"}};
  for (const LdCheck& c : lds)
    if (int e = check_ld(c.ld, c.heads, head_dim, c.what)) return e;
  FH_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv && workspace,
             "attn_bwd: null pointer");
  FH_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) && aligned16(dout) &&
                 aligned16(dq) && aligned16(dk) && aligned16(dv) && aligned16(workspace),
             "attn_bwd: pointers must be 16-byte aligned");
  const int S = static_cast<int>(seq_len), nh = static_cast<int>(n_heads);
  const int nkv = static_cast<int>(n_kv_heads), group = static_cast<int>(n_heads / n_kv_heads);
  // workspace: delta = rowsum(dO*O) and nl2 = -lse*log2(e) per query, both
  // written by the dQ kernel (its prologue), read by the dK/dV kernel.
  float* delta = static_cast<float*>(workspace);
  float* nl2 = delta + batch * n_heads * seq_len;
  const RopeRows<uint16_t> rb{static_cast<const uint16_t*>(rp.cos), static_cast<const uint16_t*>(rp.sin),
                              rp.per_token};
  const RopeRows<float> rf{static_cast<const float*>(rp.cos), static_cast<const float*>(rp.sin), rp.per_token};
  if (dt == FH_BF16) {
    // dQ first: its prologue writes delta = rowsum(dO*O), which dK/dV reads.
    const dim3 gq(static_cast<unsigned>((seq_len + 127) / 128), static_cast<unsigned>(batch * n_heads));
    dispatch_hd(head_dim, [&](auto hdc) {
      constexpr int HD = decltype(hdc)::value;
      hipLaunchKernelGGL((k_attn_bwd_dq<HD>), gq, dim3(256), 0, stream,
                         static_cast<const uint16_t*>(q), ldq, static_cast<const uint16_t*>(k), ldk,
                         static_cast<const uint16_t*>(v), ldv, static_cast<const uint16_t*>(o), ldo,
                         static_cast<const uint16_t*>(dout), lddo, lse, delta, nl2,
                         static_cast<uint16_t*>(dq), lddq, S, nh, group, scale * kLog2e, scale, rb);
      const auto kq = static_cast<const uint16_t*>(q);
      const auto kk = static_cast<const uint16_t*>(k);
      const auto kvp = static_cast<const uint16_t*>(v);
      const auto kg = static_cast<const uint16_t*>(dout);
      const auto kdk = static_cast<uint16_t*>(dk);
      const auto kdv = static_cast<uint16_t*>(dv);
      if constexpr (HD <= 64) {
        using DT = DkdvFusedTiles<HD>;
        const int64_t nkb = (seq_len + DT::NWH * 32 - 1) / (DT::NWH * 32);
        const dim3 gk(static_cast<unsigned>((nkb + 1) / 2), static_cast<unsigned>(batch * n_kv_heads));
        hipLaunchKernelGGL((k_attn_bwd_dkdv_fused<HD>), gk, dim3(DT::NT), 0, stream, kq, ldq, kk,
                           ldk, kvp, ldv, kg, lddo, nl2, delta, kdk, lddk, kdv, lddv, S, nh, nkv,
                           group, scale * kLog2e, scale, rb);
      } else {
        using DT = DkdvTiles<HD>;
        const int64_t nkb = (seq_len + DT::NKS * 32 - 1) / (DT::NKS * 32);
        const dim3 gk(static_cast<unsigned>(nkb), static_cast<unsigned>(batch * n_kv_heads));
        hipLaunchKernelGGL((k_attn_bwd_dkdv<HD>), gk, dim3(DT::NT), 0, stream, kq, ldq, kk, ldk,
                           kvp, ldv, kg, lddo, nl2, delta, kdk, lddk, kdv, lddv, S, nh, nkv, group,
                           scale * kLog2e, scale, rb);
      }
      return 0;
    });
  } else {
    const int64_t tokens = batch * seq_len;
    const unsigned dblocks = static_cast<unsigned>((tokens * n_heads + 255) / 256);
    hipLaunchKernelGGL((k_attn_delta<float>), dim3(dblocks), dim3(256), 0, stream,
                       static_cast<const float*>(o), ldo, static_cast<const float*>(dout), lddo,
                       delta, S, nh, static_cast<int>(head_dim), tokens);
    const int64_t qrows = batch * n_heads * seq_len, krows = batch * n_kv_heads * seq_len;
    dispatch_hd(head_dim, [&](auto hdc) {
      hipLaunchKernelGGL((k_attn_bwd_dq_f32<hdc()>), dim3(static_cast<unsigned>((qrows + 127) / 128)),
                         dim3(128), 0, stream, static_cast<const float*>(q), ldq,
                         static_cast<const float*>(k), ldk, static_cast<const float*>(v), ldv,
                         static_cast<const float*>(dout), lddo, lse, delta, static_cast<float*>(dq),
                         lddq, S, nh, group, scale, qrows, rf);
      hipLaunchKernelGGL((k_attn_bwd_dkdv_f32<hdc()>), dim3(static_cast<unsigned>((krows + 127) / 128)),
                         dim3(128), 0, stream, static_cast<const float*>(q), ldq,
                         static_cast<const float*>(k), ldk, static_cast<const float*>(v), ldv,
                         static_cast<const float*>(dout), lddo, lse, delta,
                         static_cast<float*>(dk), lddk, static_cast<float*>(dv), lddv, S, nh, nkv,
                         group, scale, krows, rf);
      return 0;
    });
  }
  return check_launch(rp.cos ? "fh_attn_bwd_rope" : "fh_attn_bwd");
}

}  // namespace

extern "C" int fh_attn_bwd(fh_dtype dt, const void* q, int64_t ldq, const void* k, int64_t ldk,
                           const void* v, int64_t ldv, const void* o, int64_t ldo,
                           const void* dout, int64_t lddo, const float* lse, void* dq,
                           int64_t lddq, void* dk, int64_t lddk, void* dv, int64_t lddv,
                           void* workspace, int64_t batch, int64_t seq_len, int64_t n_heads,
                           int64_t n_kv_heads, int64_t head_dim, float scale, hipStream_t stream) {
  return attn_bwd_impl(dt, q, ldq, k, ldk, v, ldv, o, ldo, dout, lddo, lse, dq, lddq, dk, lddk, dv, lddv,
                       workspace, batch, seq_len, n_heads, n_kv_heads, head_dim, scale,
                       RopeArgs{nullptr, nullptr, 0}, stream);
}

extern "C" int fh_attn_bwd_rope(fh_dtype dt, const void* q, int64_t ldq, const void* k, int64_t ldk,
                                const void* v, int64_t ldv, const void* o, int64_t ldo,
                                const void* dout, int64_t lddo, const float* lse, void* dq,
                                int64_t lddq, void* dk, int64_t lddk, void* dv, int64_t lddv,
                                void* workspace, int64_t batch, int64_t seq_len, int64_t n_heads,
                                int64_t n_kv_heads, int64_t head_dim, float scale, const void* cos,
                                const void* sin, int cos_per_token, hipStream_t stream) {
  FH_REQUIRE(cos && sin, "attn_bwd_rope: null cos/sin");
  FH_REQUIRE(aligned16(cos) && aligned16(sin), "attn_bwd_rope: cos/sin must be 16-byte aligned");
  return attn_bwd_impl(dt, q, ldq, k, ldk, v, ldv, o, ldo, dout, lddo, lse, dq, lddq, dk, lddk, dv, lddv,
                       workspace, batch, seq_len, n_heads, n_kv_heads, head_dim, scale,
                       RopeArgs{cos, sin, cos_per_token ? 1 : 0}, stream);
}
