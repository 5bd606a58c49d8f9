// Device-side building blocks shared by the gfx950 kernels of libh3attn.
//
// MFMA fragment conventions (v_mfma_f32_32x32x16_bf16, one 64-lane wave):
//   A operand (32 x 16, M x K): lane l holds A[l%32][k-slot (l/32, e)], e = 0..7
//   B operand (16 x 32, K x N): lane l holds B[k-slot (l/32, e)][l%32]
//   C/D (32 x 32, 16 fp32 per lane): lane l, register r holds
//        C[8*(r/4) + 4*(l/32) + r%4][l%32]
// A and B pair their k-slots by (l/32, e), so any assignment of the 16
// contraction indices to slots works as long as A and B agree.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "h3a_queue.h"

namespace h3a {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ f32x16 mfma_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Two fp32 -> packed bf16 pair (round to nearest even; v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Value held by the lane 32 positions away (lanes l and l^32 exchange):
// combine(x) over the pair is op(pair.x, pair.y) on both halves.
__device__ __forceinline__ float half_swap_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_swap_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Raw buffer resource (V#) over `rows` rows of `stride` elements, each row
// holding 128 bf16: num_records is the exact byte extent, so any access past
// the last valid row returns zeros.  Word 3 is the gfx9-family default config.
constexpr int kBufferConfig = 0x00020000;
// Strides are below 2^24 elements and rows at most 128 (checked by the
// entry points), so the byte extent is computed in 32 bits.
__device__ __forceinline__ uint32_t stage_bytes(int64_t stride, int rows) {
  return rows > 0 ? ((uint32_t)(rows - 1) * (uint32_t)stride + 128u) * 2u : 0u;
}

// base + key0 * stride elements, for 0 <= key0 and 0 <= stride < 2^24: one
// unsigned 32x32 -> 64-bit multiply instead of a signed 64-bit one.
__device__ __forceinline__ const uint16_t *stage_ptr(const uint16_t *base, int key0, int64_t stride) {
  return base + (uint64_t)(uint32_t)key0 * (uint32_t)stride;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t stage_rsrc(const uint16_t *base, int64_t stride,
                                                             int rows) {
  const uint32_t bytes = stage_bytes(stride, rows);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(base), (short)0, (int)bytes,
                                           kBufferConfig);
}

__device__ __forceinline__ u32x4 buffer_load_b128(__amdgpu_buffer_rsrc_t res, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(res, (int)byte_off, 0, 0);
}

// LDS DMA (buffer_load_dwordx4 ... lds): each lane's 16 bytes at `byte_off`
// go straight to LDS at lds_dst + 16 * lane, with no VGPR staging.  lds_dst
// must be wave-uniform (it is passed in M0).  Lanes past the resource's range
// write zeros.  Completion is counted by vmcnt like any vector-memory load.
//
// Issued as inline asm on purpose: the compiler cannot tell which LDS bytes a
// DMA writes, and with the builtin it waits for every DMA in flight before
// any later LDS read, including reads of the other buffer.  The caller owns
// completion: a vmcnt wait (wait_vmem_le) and a barrier before the LDS
// bytes are read.
// The compiler's own vmcnt waits stay correct, since extra loads issued
// after one of its loads only make a wait for that load more conservative.
// `desc` is the V# as four scalar words (stage_desc); `m0` is the LDS byte
// address of the destination (lds_address).
__device__ __forceinline__ void buffer_load_lds_b128(u32x4 desc, uint32_t byte_off, uint32_t m0) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(byte_off), "s"(desc), "{m0}"(m0)
               : "memory");
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_address(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// x + IMM on the scalar unit, opaque to the compiler: a wave-uniform cursor
// advanced in place cannot be folded into per-use constants that the
// compiler would then keep live across a loop.
template <uint32_t IMM>
__device__ __forceinline__ uint32_t opaque_sadd(uint32_t x) {
  uint32_t r;
  asm volatile("s_add_u32 %0, %1, %2" : "=s"(r) : "s"(x), "i"(IMM) : "scc");
  return r;
}

// stage_rsrc's V# as four words for inline asm: base address (48 bits, stride
// 0), num_records, config.  Each word goes through readfirstlane, so the
// operand is provably wave-uniform and lives in SGPRs whatever the register
// pressure around the call.
__device__ __forceinline__ u32x4 stage_desc(const uint16_t *base, int64_t stride, int rows) {
  const uint32_t bytes = stage_bytes(stride, rows);
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)addr),
               (uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)(addr >> 32) & 0xffffu)),
               (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes), (uint32_t)kBufferConfig};
}

// s_waitcnt vmcnt(N): at most the N most recent vector-memory loads of this
// wave (LDS DMA included) are still in flight; loads complete in order.  The
// other counters are left alone (expcnt 7, lgkmcnt 15).
template <int N>
__device__ __forceinline__ void wait_vmem_le() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_vmem_all() { wait_vmem_le<0>(); }

// ds_read_b64_tr_b16 (LDS transpose read).  Within each group of 16 lanes,
// lane j receives element j%4 of the 4 consecutive 16-bit values addressed by
// lanes 4k + j/4, for k = 0..3 (result element k).  `p` must point into LDS.
__device__ __forceinline__ u32x2 lds_read_tr16_b64(const uint16_t *p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 *lds_s16x4_ptr;
  const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(const_cast<uint16_t *>(p)));
  return __builtin_bit_cast(u32x2, r);
}

// acc + lo(w) + hi(w) for a packed bf16 pair (v_dot2 with (1, 1)).
__device__ __forceinline__ float dot2_bf16_ones(uint32_t w, float acc) {
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one, acc, false);
}

// xcd_remap (the XCD-aware deal of work items) lives in h3a_queue.h.

}  // namespace h3a
