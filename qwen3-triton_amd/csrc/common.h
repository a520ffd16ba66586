// Shared device helpers for the gfx950 (CDNA4) kernels of libq3hip.
//
// Conventions used by every kernel in this library:
//  * wavefront = 64 lanes; reductions use DPP row ops and cross-row swizzles;
//  * HBM traffic moves in 16-byte vectors (8 x 16-bit or 4 x fp32 elements);
//  * arithmetic is fp32 internally and every output is rounded exactly once.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/q3hip.h"

#define Q3_DEV __device__ __forceinline__

typedef unsigned short u16;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;   // MFMA operand (8 x bf16)
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

// ------------------------------------------------------------------ scalar conversions
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
Q3_DEV float bf16_to_f32(u16 h) { return __uint_as_float(((uint32_t)h) << 16); }
// fp32 -> bf16 with IEEE round-to-nearest-even: one v_cvt_pk_bf16_f32 (gfx950 hardware convert).
Q3_DEV u16 f32_to_bf16(float f) { return __builtin_bit_cast(u16, (__bf16)f); }
// Two fp32 -> packed bf16 pair (lo in bits 0..15) in a single v_cvt_pk_bf16_f32.
Q3_DEV uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
Q3_DEV float f16_to_f32(u16 h) { return (float)__builtin_bit_cast(_Float16, h); }
Q3_DEV u16 f32_to_f16(float f) { return __builtin_bit_cast(u16, (_Float16)f); }

// Element type tags.  `storage` is the in-memory type; load/store go through fp32.
struct F32 { typedef float storage; static constexpr int vec = 4; static constexpr int code = Q3_F32; };
struct F16 { typedef u16 storage; static constexpr int vec = 8; static constexpr int code = Q3_F16; };
struct BF16 { typedef u16 storage; static constexpr int vec = 8; static constexpr int code = Q3_BF16; };

template <typename T> Q3_DEV float to_f32(typename T::storage v);
template <> Q3_DEV float to_f32<F32>(float v) { return v; }
template <> Q3_DEV float to_f32<F16>(u16 v) { return f16_to_f32(v); }
template <> Q3_DEV float to_f32<BF16>(u16 v) { return bf16_to_f32(v); }
template <typename T> Q3_DEV typename T::storage from_f32(float v);
template <> Q3_DEV float from_f32<F32>(float v) { return v; }
template <> Q3_DEV u16 from_f32<F16>(float v) { return f32_to_f16(v); }
template <> Q3_DEV u16 from_f32<BF16>(float v) { return f32_to_bf16(v); }

// Two values of a 16-bit type packed into one 32-bit word (lo in bits 0..15).
template <typename T> Q3_DEV uint32_t pack2(float lo, float hi) {
  return (uint32_t)from_f32<T>(lo) | ((uint32_t)from_f32<T>(hi) << 16);
}
template <> Q3_DEV uint32_t pack2<BF16>(float lo, float hi) { return pack_bf16x2(lo, hi); }

// One 16-byte vector unpacked to fp32: VEC = 8 for 16-bit types, 4 for fp32.
template <typename T> struct Vec { float v[T::vec]; };

// 16 bytes of storage (T::vec elements) as floats.
template <typename T> Q3_DEV Vec<T> unpack_vec(i32x4 raw) {
  Vec<T> r;
  if constexpr (T::vec == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) r.v[i] = __int_as_float(raw[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t w = (uint32_t)raw[i];
      r.v[2 * i] = to_f32<T>((u16)(w & 0xffffu));
      r.v[2 * i + 1] = to_f32<T>((u16)(w >> 16));
    }
  }
  return r;
}
template <typename T> Q3_DEV Vec<T> load_vec(const typename T::storage* p) {
  return unpack_vec<T>(*reinterpret_cast<const i32x4*>(p));
}
template <typename T> Q3_DEV void store_vec(typename T::storage* p, const Vec<T>& r) {
  i32x4 raw;
  if constexpr (T::vec == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) raw[i] = __float_as_int(r.v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) raw[i] = (int)pack2<T>(r.v[2 * i], r.v[2 * i + 1]);
  }
  *reinterpret_cast<i32x4*>(p) = raw;
}

// ------------------------------------------------------------------ streaming access
// Streaming operands are touched once: non-temporal loads and stores keep them out of the caches.
Q3_DEV i32x4 ld_nt(const void* p) { return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p)); }
template <typename T> Q3_DEV void st_nt(typename T::storage* p, const Vec<T>& r) {
  i32x4 raw;
  if constexpr (T::vec == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) raw[i] = __float_as_int(r.v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) raw[i] = (int)pack2<T>(r.v[2 * i], r.v[2 * i + 1]);
  }
  __builtin_nontemporal_store(raw, reinterpret_cast<i32x4*>(p));
}

// ------------------------------------------------------------------ matrix cores
// D(16x16, fp32) += A(16x32) B(32x16), 16-bit inputs: lane l holds A[l % 16][8 (l / 16) + 0..7],
// B[8 (l / 16) + 0..7][l % 16] and D[4 (l / 16) + 0..3][l % 16].
template <typename T> Q3_DEV f32x4 mfma_16x16x32(bf16x8_t a, bf16x8_t b, f32x4 c);
template <> Q3_DEV f32x4 mfma_16x16x32<BF16>(bf16x8_t a, bf16x8_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
template <> Q3_DEV f32x4 mfma_16x16x32<F16>(bf16x8_t a, bf16x8_t b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                 0, 0, 0);
}

// ------------------------------------------------------------------ wave64 reductions
// Butterfly over aligned groups of WIDTH lanes (WIDTH a power of two <= 64); every lane in
// the group ends with the full result.  Offsets 1/2 use DPP quad permutes, 4/8 DPP row
// mirrors (valid after the previous steps made the group uniform), 16/32 use swizzles.
template <int WIDTH> Q3_DEV float group_sum(float x) {
  if constexpr (WIDTH >= 2)
    x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true));
  if constexpr (WIDTH >= 4)
    x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true));
  if constexpr (WIDTH >= 8)
    x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true));
  if constexpr (WIDTH >= 16)
    x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x140, 0xF, 0xF, true));
  if constexpr (WIDTH >= 32) x += __shfl_xor(x, 16, 64);
  if constexpr (WIDTH >= 64) x += __shfl_xor(x, 32, 64);
  return x;
}
template <int WIDTH> Q3_DEV float group_max(float x) {
#pragma unroll
  for (int o = 1; o < WIDTH; o <<= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}

Q3_DEV int lane_id() { return (int)(threadIdx.x & 63); }

// sigmoid(g) = 1 / (1 + e^-g) with the hardware exp2 and reciprocal (SiLU(g) = g * q3_sigmoid(g)).
Q3_DEV float q3_sigmoid(float g) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

// Launch helpers: every entry point returns the launch status as an int.
#define Q3_CHECK_LAUNCH() return (int)hipGetLastError()
#define Q3_REQUIRE(cond) \
  do {                   \
    if (!(cond)) return Q3_ERR_INVALID; \
  } while (0)

// Grid size for grid-stride elementwise kernels: enough workgroups to fill 256 CUs x 8 waves.
static inline unsigned q3_grid_for(int64_t work_items, int block) {
  int64_t g = (work_items + block - 1) / block;
  if (g > 256 * 32) g = 256 * 32;
  if (g < 1) g = 1;
  return (unsigned)g;
}
