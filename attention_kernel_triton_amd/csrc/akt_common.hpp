// Shared device helpers for the gfx950 attention kernels.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, MFMA
// f16 shapes with the doubled K depth (16x16x32, 32x32x16), and the
// v_permlane{16,32}_swap lane exchanges.  There is no other target.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace akt {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// MFMA wrappers.  Operand convention used by every kernel in this library:
//   A[m][k]: lane = m + M * g, element e   (g = lane / M)
//   B[k][n]: lane = n + N * g, element e
// where the reduction index k is the same function k(g, e) for A and B, so a
// kernel may assign any physical index (head dim, key slot) to (g, e) as long
// as both operands use the same assignment.
//   16x16 result: lane = n + 16 * (m / 4), register m % 4
//   32x32 result: lane = n + 32 * ((m / 4) % 2), register (m % 4) + 4 * (m / 8)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float16_t mfma32x32x16_bf16(bf16x8_t a, bf16x8_t b, float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Cross-lane helpers.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}
__device__ __forceinline__ float shfl_f(float v, int src) { return __shfl(v, src, kWave); }
__device__ __forceinline__ uint32_t shfl_u(uint32_t v, int src) {
  return (uint32_t)__shfl((int)v, src, kWave);
}

// Exchange with lane l ^ 32 / l ^ 16 through v_permlane32_swap /
// v_permlane16_swap (no LDS round trip).  Swapping a register with itself
// yields, in each lane, the pair {x[l], x[l ^ 32]} (or x[l ^ 16]) in some
// order, so any commutative combine of the two results is the butterfly.
__device__ __forceinline__ void swap32(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void swap16(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

// Lane h of each 16-lane row, broadcast to the whole row (DPP row_newbcast:
// one VALU move, no LDS round trip).  h must fold to a constant.
template <int H>
__device__ __forceinline__ uint32_t row_bcast_c(uint32_t v) {
  static_assert(H >= 0 && H < 16, "row lane");
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x150 + H, 0xf, 0xf, false);
}
__device__ __forceinline__ uint32_t row_bcast(uint32_t v, int h) {
  switch (h) {
    case 0: return row_bcast_c<0>(v);
    case 1: return row_bcast_c<1>(v);
    case 2: return row_bcast_c<2>(v);
    case 3: return row_bcast_c<3>(v);
    case 4: return row_bcast_c<4>(v);
    case 5: return row_bcast_c<5>(v);
    case 6: return row_bcast_c<6>(v);
    case 7: return row_bcast_c<7>(v);
    case 8: return row_bcast_c<8>(v);
    case 9: return row_bcast_c<9>(v);
    case 10: return row_bcast_c<10>(v);
    case 11: return row_bcast_c<11>(v);
    case 12: return row_bcast_c<12>(v);
    case 13: return row_bcast_c<13>(v);
    case 14: return row_bcast_c<14>(v);
    default: return row_bcast_c<15>(v);
  }
}
__device__ __forceinline__ float row_bcast_f(float v, int h) {
  return __uint_as_float(row_bcast(__float_as_uint(v), h));
}

// Max / sum over the two 32-lane halves of the wave (lane l and l ^ 32).
__device__ __forceinline__ float xor32_max(float v) {
  float a, b;
  swap32(v, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float xor32_sum(float v) {
  float a, b;
  swap32(v, a, b);
  return a + b;
}

// Reduce across the four 16-lane rows (l ^ 16, l ^ 32).
__device__ __forceinline__ float rows_max(float v) {
  float a, b;
  swap16(v, a, b);
  return xor32_max(fmaxf(a, b));
}
__device__ __forceinline__ float rows_sum(float v) {
  float a, b;
  swap16(v, a, b);
  return xor32_sum(a + b);
}

// ---------------------------------------------------------------------------
// Arithmetic helpers.
// ---------------------------------------------------------------------------
// Hardware base-2 exponential (v_exp_f32).  exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// fp32 pair -> packed fp16 pair (round to nearest even).
__device__ __forceinline__ uint32_t pack_half2(float lo, float hi) {
  half2_t h = {(half_t)lo, (half_t)hi};
  return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ half2_t as_half2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

// c + a.x * b.x + a.y * b.y with fp32 accumulation (v_dot2_f32_f16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_half2(a), as_half2(b), c, false);
}

// fp32 pair -> packed bf16 pair (round to nearest even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float float2_v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2_v{lo, hi}, bf16x2_t));
}
// c + a.x * b.x + a.y * b.y for bf16 pairs with fp32 accumulation (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Pair up two fp16 words from two registers: lo16(a) | lo16(b) << 16.
__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
// hi16(a) | hi16(b) << 16.
__device__ __forceinline__ uint32_t pair_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

__device__ __forceinline__ half8_t as_half8(uint4_t u) { return __builtin_bit_cast(half8_t, u); }
__device__ __forceinline__ uint4_t as_uint4(half8_t h) { return __builtin_bit_cast(uint4_t, h); }
__device__ __forceinline__ float4_t as_float4u(uint4_t u) { return __builtin_bit_cast(float4_t, u); }
__device__ __forceinline__ uint4_t as_uint4f(float4_t f) { return __builtin_bit_cast(uint4_t, f); }

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4;

// ds_read_b64_tr_b16: within each 16-lane group, output lane i, element j is
// component (i % 4) of the 8-byte chunk addressed by source lane 4j + i / 4.
// If source lane s addresses row k0 + s / 4, columns c0 + 4 (s % 4) .. +3 of a
// row-major fp16 matrix, output lane i receives rows k0..k0+3 of column c0 + i.
__device__ __forceinline__ uint2 ds_read_tr16(const void* lds_ptr) {
  const short4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(lds_ptr));
  return __builtin_bit_cast(uint2, r);
}

// 16-byte global load / store.
__device__ __forceinline__ uint4_t ld16(const void* p) {
  return *reinterpret_cast<const uint4_t*>(p);
}
__device__ __forceinline__ void st16(void* p, uint4_t v) { *reinterpret_cast<uint4_t*>(p) = v; }

// 64-bit LDS word shared by the waves of a workgroup, read and written whole.
// Relaxed workgroup-scope atomics keep the LDS address space: a volatile
// access through a generic pointer becomes a flat access, and the wait for
// one of those also waits for every global load the wave has in flight.
__device__ __forceinline__ void lds_store_u64(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ unsigned long long lds_load_u64(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Readfirstlane for 32-bit ints: moves a wave-uniform value into an SGPR.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// ---------------------------------------------------------------------------
// Device-coherent 16-byte accesses through a raw buffer resource.
// ---------------------------------------------------------------------------
// Word 3 of a raw (stride 0) gfx9 buffer resource: 32-bit data format.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of the buffer intrinsics: the device-scope bit (sc1).
// A device-scope store is acknowledged only once it is visible to every CU of
// the device, whichever XCD (and L2) it belongs to; a device-scope load never
// returns a line that another XCD's L2 has made stale.  These are the
// accesses the compiler emits for relaxed agent-scope atomics, here 16 bytes
// wide.
constexpr int kScopeDevice = 16;

// 16-byte device-scope store / load at byte offset `off` (< 2^31) from `base`.
__device__ __forceinline__ void st16_device(void* base, uint32_t off, uint4_t v) {
  const auto r = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, kBufferWord3);
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kScopeDevice);
}
__device__ __forceinline__ uint4_t ld16_device(const void* base, uint32_t off) {
  const auto r = __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, 0x7fffffff, kBufferWord3);
  return __builtin_bit_cast(uint4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kScopeDevice));
}

}  // namespace akt
