// Shared device helpers for the gfx950 W4A16 MoE kernels.
//
// Packed int4 layout (compressed-tensors "pack-quantized", the reference's
// hybrid_agent/quantization.py:132-137): int32 word p[n, j] holds
// w[n, 8j+i] for i = 0..7 in bits 4i..4i+3 as offset binary u = q + 8.
//
// Every kernel dequantises exactly: each weight becomes bf16_RNE((u - 8) * s),
// bit-identical to the reference's dequantize_int4_packed, and enters a bf16
// MFMA with fp32 accumulation -- the reference's dequantise-then-matmul.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a16 {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

// f32 -> bf16 bits, round to nearest even (lowers to v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v;
  v.x = (__bf16)lo;
  v.y = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

// p[i] for a wavefront-uniform i, through the scalar data cache (a read of
// the constant address space): scalar loads are counted apart from vector
// loads, so the value arrives without waiting for vector loads in flight.
// Only for data no thread of the running kernel writes.
__device__ __forceinline__ int32_t ld_uniform(const int32_t* p, int i) {
  typedef __attribute__((address_space(4))) const int32_t cint32_t;
  return ((cint32_t*)p)[__builtin_amdgcn_readfirstlane(i)];
}

// Hides a value from constant folding so it stays in a register.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Exact dequantization constants of one group scale s (see unpack_exact).
struct ExactScale {
  float s, c0, c1;
};

__device__ __forceinline__ ExactScale exact_scale(float s) {
  return ExactScale{s, -1032.0f * s, -72.0f * s};
}

// Registers the exact unpack works with: gfx9 VOP3 instructions take no
// literal operands, so the masks and the two fp16 exponents live in
// registers and each fp16 pair is one v_and_or_b32.
struct ExactRegs {
  uint32_t m0, m1, magic0, magic1;
};

__device__ __forceinline__ ExactRegs exact_regs() {
  return ExactRegs{opaque(0x000F000Fu), opaque(0x00F000F0u), opaque(0x64006400u), opaque(0x54005400u)};
}

// Exact unpack of one packed word with scale s: 8 values bf16_RNE((u-8)*s).
// PAIRED selects the element order: natural (k = 0..7) or (0,4,1,5,2,6,3,7),
// the order in which the decode gate_up epilogue writes intermediate rows.
//
// Each nibble becomes an fp16 by OR-ing it into the mantissa of an fp16
// whose ulp is 1 at the nibble's place: nibbles 0/4 and 2/6 (the latter after
// >> 8) sit at mantissa bits 0..3 under exponent 2^10 (0x6400) and read
// 1024 + u; nibbles 1/5 and 3/7 sit at bits 4..7 under exponent 2^6 (0x5400)
// and read 64 + u.  One v_fma_mix_f32 per value then takes the fp16 half
// straight into an fp32 fma:
//   (1024 + u) * s - 1032 s = (u - 8) s
//   (64 + u)   * s - 72 s   = (u - 8) s
// The products are exact inside the fma and 1032 s, 72 s are exact in fp32
// (s has 8 significant bits, 1032 and 72 have two set bits each), so the
// single rounding returns (u-8)*s exactly, which v_cvt_pk_bf16_f32 rounds to
// bf16 (RNE).  Valid for |s| < 2^118, where 1032 s stays finite (bf16 group
// scales of quantized weights are far below).
template <bool PAIRED>
__device__ __forceinline__ u32x4_t unpack_exact(uint32_t w, const ExactScale& es, const ExactRegs& k) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  const uint32_t w8 = w >> 8;
  const f16x2_t p0 = __builtin_bit_cast(f16x2_t, (w & k.m0) | k.magic0);   // 1024 + u0, u4
  const f16x2_t p1 = __builtin_bit_cast(f16x2_t, (w & k.m1) | k.magic1);   // 64 + u1, u5
  const f16x2_t p2 = __builtin_bit_cast(f16x2_t, (w8 & k.m0) | k.magic0);  // 1024 + u2, u6
  const f16x2_t p3 = __builtin_bit_cast(f16x2_t, (w8 & k.m1) | k.magic1);  // 64 + u3, u7
  const float v0 = __builtin_fmaf((float)p0.x, es.s, es.c0);
  const float v4 = __builtin_fmaf((float)p0.y, es.s, es.c0);
  const float v1 = __builtin_fmaf((float)p1.x, es.s, es.c1);
  const float v5 = __builtin_fmaf((float)p1.y, es.s, es.c1);
  const float v2 = __builtin_fmaf((float)p2.x, es.s, es.c0);
  const float v6 = __builtin_fmaf((float)p2.y, es.s, es.c0);
  const float v3 = __builtin_fmaf((float)p3.x, es.s, es.c1);
  const float v7 = __builtin_fmaf((float)p3.y, es.s, es.c1);
  u32x4_t r;
  if (PAIRED) {
    r.x = pack_bf16x2(v0, v4);
    r.y = pack_bf16x2(v1, v5);
    r.z = pack_bf16x2(v2, v6);
    r.w = pack_bf16x2(v3, v7);
  } else {
    r.x = pack_bf16x2(v0, v1);
    r.y = pack_bf16x2(v2, v3);
    r.z = pack_bf16x2(v4, v5);
    r.w = pack_bf16x2(v6, v7);
  }
  return r;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Raw buffer access (gfx9 descriptor: 32-bit data format, no stride).  The
// base and size live in SGPRs when wave-uniform; each lane supplies a 32-bit
// byte offset; reads past num_bytes return zero.
constexpr int kBufferRsrcWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_bytes,
                                           kBufferRsrcWord3);
}

__device__ __forceinline__ u32x4_t buf_ld16(__amdgpu_buffer_rsrc_t r, int voff, int imm) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff + imm, 0, 0));
}

__device__ __forceinline__ uint16_t buf_ld_u16(__amdgpu_buffer_rsrc_t r, int voff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0);
}

// 16-byte global load / store helpers.
__device__ __forceinline__ u32x4_t ld16(const void* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4_t v) {
  *reinterpret_cast<u32x4_t*>(p) = v;
}

// All-lane wavefront reductions through DPP, no LDS round trips: a
// butterfly inside each 16-lane row (quad swaps, then row rotations by 4 and
// 8), then the four row results combined from v_readlane.  Every lane gets
// the result.
template <typename Op>
__device__ __forceinline__ uint32_t dpp_row_reduce(uint32_t v, Op op) {
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xF, 0xF, false));  // row_ror:4
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false));  // row_ror:8
  return v;
}

template <typename Op>
__device__ __forceinline__ uint32_t dpp_wave_reduce(uint32_t v, Op op) {
  v = dpp_row_reduce(v, op);
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return op(op(r0, r1), op(r2, r3));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return dpp_wave_reduce(v, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
}

__device__ __forceinline__ float wave_max_f32(float v) {
  return __uint_as_float(dpp_wave_reduce(__float_as_uint(v), [](uint32_t x, uint32_t y) {
    return __float_as_uint(fmaxf(__uint_as_float(x), __uint_as_float(y)));
  }));
}

__device__ __forceinline__ float wave_sum_f32(float v) {
  return __uint_as_float(dpp_wave_reduce(__float_as_uint(v), [](uint32_t x, uint32_t y) {
    return __float_as_uint(__uint_as_float(x) + __uint_as_float(y));
  }));
}

// gelu_pytorch_tanh, 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3),
// evaluated through the identity 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)) in
// fp32 (one exponential, one reciprocal; exact limits -0 and x for large |x|).
__device__ __forceinline__ float gelu_tanh_f32(float x) {
  const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  return __fdividef(x, 1.0f + __expf(-2.0f * u));
}

// Value of the lane 8 positions away inside the 16-lane row (j <-> j ^ 8),
// through DPP row rotation.
__device__ __forceinline__ float lane_xor8(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
}

}  // namespace w4a16
