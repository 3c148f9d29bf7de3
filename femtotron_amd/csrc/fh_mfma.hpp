// MFMA tile helpers shared by the attention and GEMM kernels (gfx950, wave64).
//
// v_mfma_f32_32x32x16_bf16: lane i of an operand holds row/col i%32 and the
// K-slice 8*(i/32)..+7; lane i of the fp32 accumulator holds column i%32 and
// rows 8*(j/4) + 4*(i/32) + j%4, j = 0..15.
//
// LDS tiles are [rows x HD] bf16 without padding, XOR-swizzled in 16-byte
// chunks: chunk c of row r is stored at chunk position c ^ swz(r).  Operands
// read a tile in two patterns, (a) ds_read_b128 of one chunk from 16
// consecutive rows and (b) ds_read_b64_tr_b16 of 4 consecutive chunks from 4
// consecutive rows (first row a multiple of 4) across 32 lanes; swz() maps
// both onto the 16 distinct 4-bank groups of one LDS cycle, so neither has
// bank conflicts.  A read address is a per-lane constant XOR a compile-time
// constant, plus an immediate offset.
#pragma once

#include "fh_common.hpp"

namespace fh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int j = 0; j < 16; ++j) z[j] = 0.f;
  return z;
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// ------------------------------------------------------------- LDS tiles
template <int HD>
__device__ __forceinline__ int swz(int r) {
  if constexpr (HD == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
  else if constexpr (HD == 64) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else return (r >> 2) & 3;
}

// Pattern (a) lane constant: row lane%32 of a 32-row group, chunk lane/32.
// Step s (K = 16s..16s+15 along the row) of the group at row0 is read at byte
// row0*2*HD + (A ^ 32s).
template <int HD>
__device__ __forceinline__ int lane_off_a(int lane) {
  const int l32 = lane & 31, hl = lane >> 5;
  return l32 * (2 * HD) + ((hl ^ swz<HD>(l32)) << 4);
}

// Pattern (b) lane constant for rows 4*(lane/32) + (lane%16)/4 (+ plus8):
// the 32-column block dt of the 16-row group at row0 is read at byte
// row0*2*HD + (B ^ 64dt).
template <int HD>
__device__ __forceinline__ int lane_off_b(int lane, int plus8) {
  const int hl = lane >> 5, L = lane & 15, mh = (lane >> 4) & 1;
  const int r = 4 * hl + (L >> 2) + plus8;
  const int cb = 2 * mh + ((L & 3) >> 1);
  return r * (2 * HD) + ((cb ^ swz<HD>(r)) << 4) + 8 * (L & 1);
}

// Makes the per-lane read offsets opaque to the optimizer once per loop
// iteration, so that their XORs with compile-time constants are recomputed
// (one VALU op per read) instead of each being kept live in its own register.
__device__ __forceinline__ void refresh_offsets(int& a, int& b0, int& b8) {
  asm volatile("" : "+v"(a), "+v"(b0), "+v"(b8));
}

// Operand with K along the rows of a swizzled tile: lane i gets row
// row0 + i%32, columns 16s + 8*(i/32) .. +7.
template <int HD>
__device__ __forceinline__ bf16x8 lds_frag(const char* tile, int a_off, int row0, int s) {
  return *reinterpret_cast<const bf16x8*>(tile + row0 * (2 * HD) + (a_off ^ (32 * s)));
}

// Operand with K down the rows of a swizzled tile X: lane i gets
// X[row0 + {4h+0..3, 8+4h+0..3}][32dt + i%32], h = i/32.
template <int HD>
__device__ __forceinline__ bf16x8 lds_frag_tr(const char* tile, int b0, int b8, int row0, int dt) {
  const char* t = tile + row0 * (2 * HD);
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + (b0 ^ (64 * dt))));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(t + (b8 ^ (64 * dt))));
  const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
  return as_bf16x8(make_uint4(ua.x, ua.y, ub.x, ub.y));
}

// acc + the sum of the 8 bf16 values of v: four v_dot2 with (1, 1), half the
// instructions of adding the 8 values unpacked.
__device__ __forceinline__ float sum_bf16x8(bf16x8 v, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const uint4 u = __builtin_bit_cast(uint4, v);
  const bf16x2 one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.x), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.y), one, acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.z), one, acc, false);
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u.w), one, acc, false);
}

// Row (M index) of accumulator entry j for lane half hl.
__device__ __forceinline__ int acc_row(int j, int hl) { return 8 * (j >> 2) + 4 * hl + (j & 3); }

// Direct-to-LDS load of rows r0 .. r0+ROWS-1 of a bf16 [*, HD] matrix (row
// stride ld elements) into a swizzled [ROWS x HD] LDS tile, shared by the NW
// waves of a block: each global_load_lds_dwordx4 fills one 1 KB run of the
// tile (RPR consecutive rows), lane i its 16-byte slot i, so the lane reads
// the global chunk that the swizzle stores in that slot.  Rows past `last`
// re-read row `last`.  The LDS writes complete asynchronously: each wave
// waits for its own loads (s_waitcnt vmcnt) before the barrier that hands
// the tile to the other waves.
template <int ROWS, int HD, int NW>
__device__ __forceinline__ void dma_tile(const uint16_t* src, int64_t ld, int r0, int last, char* dst,
                                         int wave, int lane) {
  typedef __attribute__((address_space(1))) const void* gptr;
  typedef __attribute__((address_space(3))) void* lptr;
  constexpr int CPR = HD / 8, RPR = 64 / CPR, RUNS = ROWS / RPR;
  static_assert(64 % CPR == 0 && ROWS % RPR == 0, "the tile is whole 1 KB runs");
#pragma unroll
  for (int j0 = 0; j0 < RUNS; j0 += NW) {
    const int j = j0 + wave;  // wave-uniform
    if (RUNS % NW == 0 || j < RUNS) {
      const int r = j * RPR + lane / CPR, c = (lane % CPR) ^ swz<HD>(r);
      const int64_t row = min(r0 + r, last);
      __builtin_amdgcn_global_load_lds((gptr)(src + row * ld + c * 8), (lptr)(dst + j * 1024), 16, 0, 0);
    }
  }
}

// One 1 KB direct-to-LDS copy as inline asm: lane i loads the 16 bytes at
// sbase + voff into LDS at lds + 16 i.  M0 carries the LDS address, set in the
// same statement; nothing else in these kernels uses M0, which the compiler
// reserves (hence the diagnostic it would print for the clobber).  An LDS DMA
// that reads M0 right after an SALU write of it needs one wait state (gfx9;
// the compiler puts the same s_nop before the loads it emits itself).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(uint32_t voff, const void* sbase, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}

// dma_tile with its loads as inline asm (dma16: the row base r0 in SGPRs, each
// lane's clamped row as a 32-bit offset from it; r0 <= last).  The compiler
// does not see these loads: the caller waits for them (vmcnt) itself.
template <int ROWS, int HD, int NW>
__device__ __forceinline__ void dma_tile_asm(const uint16_t* src, int64_t ld, int r0, int last, char* dst,
                                             int wave, int lane) {
  typedef __attribute__((address_space(3))) char* lptr;
  constexpr int CPR = HD / 8, RPR = 64 / CPR, RUNS = ROWS / RPR;
  static_assert(64 % CPR == 0 && ROWS % RPR == 0, "the tile is whole 1 KB runs");
  const void* base = src + static_cast<int64_t>(r0) * ld;
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lptr)dst));
#pragma unroll
  for (int j0 = 0; j0 < RUNS; j0 += NW) {
    const int j = j0 + wave;  // wave-uniform
    if (RUNS % NW == 0 || j < RUNS) {
      const int r = j * RPR + lane / CPR, c = (lane % CPR) ^ swz<HD>(r);
      const int64_t rr = min(r0 + r, last) - r0;
      dma16(static_cast<uint32_t>((rr * ld + c * 8) * 2), base, lds0 + j * 1024);
    }
  }
}

// dma16 in two statements for loops that put an MFMA between them (its issue
// is the wait state): set_m0(lds), then dma16_m0(voff, sbase).  Volatile asm
// keeps the two in order; nothing between them may write M0.
__device__ __forceinline__ void set_m0(uint32_t lds) { asm volatile("s_mov_b32 m0, %0" ::"s"(lds) : "m0"); }
__device__ __forceinline__ void dma16_m0(uint32_t voff, const void* sbase) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase) : "memory");
}
#pragma clang diagnostic pop

// dma_tile with the per-lane part of every load address computed once (init,
// outside the loop): a tile at row r0 is read at src + r0*ld, wave-uniform,
// plus this lane's fixed byte offset of each of the wave's runs, so a load
// costs no vector address arithmetic.  Only a tile that runs past `last` (the
// ragged end of a sequence) takes dma_tile's clamped path, behind a branch
// marked unlikely (as a select, both address forms were computed for every
// tile: 22 instead of 11 vector instructions per K/V block of the forward).
// Offsets are 32-bit: the caller keeps ROWS * ld * 2 below 2^32.
template <int ROWS, int HD, int NW>
struct TileDma {
  static constexpr int CPR = HD / 8, RPR = 64 / CPR, RUNS = ROWS / RPR, PER = (RUNS + NW - 1) / NW;
  uint32_t off[PER];
  __device__ __forceinline__ void init(int64_t ld, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int r = (i * NW + wave) * RPR + lane / CPR, c = (lane % CPR) ^ swz<HD>(r);
      off[i] = static_cast<uint32_t>((r * ld + c * 8) * 2);
    }
  }
  __device__ __forceinline__ void load(const uint16_t* src, int64_t ld, int r0, int last, char* dst, int wave,
                                       int lane) const {
    typedef __attribute__((address_space(1))) const void* gptr;
    typedef __attribute__((address_space(3))) void* lptr;
    if (__builtin_expect(r0 + ROWS - 1 <= last, 1)) {
      const char* base = reinterpret_cast<const char*>(src + static_cast<int64_t>(r0) * ld);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int j = i * NW + wave;  // wave-uniform
        if (RUNS % NW == 0 || j < RUNS)
          __builtin_amdgcn_global_load_lds((gptr)(base + off[i]), (lptr)(dst + j * 1024), 16, 0, 0);
      }
    } else {
      dma_tile<ROWS, HD, NW>(src, ld, r0, last, dst, wave, lane);
    }
  }
  // load() with each load issued as inline asm in its scalar-base form (the
  // row base in SGPRs, the lane's 32-bit offset in one VGPR, M0 = the LDS run):
  // no 64-bit per-lane pointers are kept.  The compiler does not see these
  // loads, so the caller must wait for them itself (wait_loads) before any
  // read of the stage, as the block loops do before their barriers.
  __device__ __forceinline__ void load_asm(const uint16_t* src, int64_t ld, int r0, int last, char* dst, int wave,
                                           int lane) const {
    typedef __attribute__((address_space(3))) char* lptr;
    if (__builtin_expect(r0 + ROWS - 1 <= last, 1)) {
      const void* base = src + static_cast<int64_t>(r0) * ld;
      const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lptr)dst));
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int j = i * NW + wave;  // wave-uniform
        if (RUNS % NW == 0 || j < RUNS) dma16(off[i], base, lds0 + j * 1024);
      }
    } else {
      dma_tile_asm<ROWS, HD, NW>(src, ld, r0, last, dst, wave, lane);
    }
  }
};

// Waits for this wave's outstanding global loads, including direct-to-LDS ones.
__device__ __forceinline__ void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Barrier for LDS data written with ds_write: waits for this wave's LDS
// operations only, not for direct-to-LDS loads still in flight into another
// buffer (a __syncthreads() would wait for those too: its workgroup release
// covers every pending LDS write).  Also a compiler barrier for memory.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace
}  // namespace fh
