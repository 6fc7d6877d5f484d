// Shared device helpers for the MoE HIP kernels (gfx950 / CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;  // bfloat16 storage
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define MOE_DEV __device__ __forceinline__

MOE_DEV float bf2f(bf16_t v) { return __uint_as_float(((uint32_t)v) << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// float -> bfloat16 with gfx950's v_cvt_pk_bf16_f32: round to nearest even,
// NaN stays NaN.
MOE_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2_t));
}
MOE_DEV bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// Elements of T in one 16-byte vector.
template <typename T> struct Vec16;
template <> struct Vec16<bf16_t> { static constexpr int N = 8; };
template <> struct Vec16<float> { static constexpr int N = 4; };

template <typename T> MOE_DEV float to_f(T v);
template <> MOE_DEV float to_f<float>(float v) { return v; }
template <> MOE_DEV float to_f<bf16_t>(bf16_t v) { return bf2f(v); }
template <typename T> MOE_DEV T from_f(float v);
template <> MOE_DEV float from_f<float>(float v) { return v; }
template <> MOE_DEV bf16_t from_f<bf16_t>(float v) { return f2bf(v); }

// 16-byte vector <-> floats
MOE_DEV void unpack16(u32x4 v, float* f, bf16_t) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
MOE_DEV void unpack16(u32x4 v, float* f, float) {
  f[0] = __uint_as_float(v.x); f[1] = __uint_as_float(v.y);
  f[2] = __uint_as_float(v.z); f[3] = __uint_as_float(v.w);
}
MOE_DEV u32x4 pack16(const float* f, bf16_t) {
  u32x4 r;
  r.x = pack_bf16x2(f[0], f[1]);
  r.y = pack_bf16x2(f[2], f[3]);
  r.z = pack_bf16x2(f[4], f[5]);
  r.w = pack_bf16x2(f[6], f[7]);
  return r;
}
MOE_DEV u32x4 pack16(const float* f, float) {
  u32x4 r;
  r.x = __float_as_uint(f[0]); r.y = __float_as_uint(f[1]);
  r.z = __float_as_uint(f[2]); r.w = __float_as_uint(f[3]);
  return r;
}

// Raw buffer resources (gfx9-family descriptor word 3).  A load whose offset
// lies beyond the resource's byte count returns zero.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOobOffset = 0x80000000u;  // beyond every resource (< 2^31 bytes)
MOE_DEV rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
MOE_DEV u32x4 buf_ld16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Pointers read from device tables are generic to the compiler; these casts
// keep their accesses on the global path (flat accesses would also count
// against the LDS wait counter).
template <typename T> MOE_DEV const __attribute__((address_space(1))) T* gptr(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}
template <typename T> MOE_DEV __attribute__((address_space(1))) T* gptr(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}

template <typename T> MOE_DEV u32x4 ld16(const T* p) { return *reinterpret_cast<const u32x4*>(p); }
template <typename T> MOE_DEV void st16(T* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

MOE_DEV float silu_f(float g) { return g / (1.0f + __expf(-g)); }
MOE_DEV float sigmoid_f(float g) { return 1.0f / (1.0f + __expf(-g)); }

// Wave-wide (64 lanes) butterfly reductions: fixed order, so bit-reproducible.
MOE_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
MOE_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Map workgroup b to a logical tile id in [0, n) so that the blocks one XCD
// receives (blocks are dealt round-robin over the 8 XCDs) form one contiguous
// range of logical tiles, and neighbouring tiles share that XCD's L2.  The
// ranges split the n tiles that exist (not the grid, which may be an upper
// bound when n depends on the routing) evenly over the XCDs, so no XCD is
// left idle by a grid larger than the work.  Returns false for blocks past
// their XCD's range; needs a grid of at least n blocks.
MOE_DEV bool xcd_slot(int b, int n, int& id) {
  const int x = b & 7, j = b >> 3, q = n >> 3, r = n & 7;
  if (j >= q + (x < r ? 1 : 0)) return false;
  id = x * q + (x < r ? x : r) + j;
  return true;
}

// Two classes of tiles, n0 of class 0 and n1 of class 1, dealt over the 8
// XCDs: each XCD receives a contiguous range of each class (neighbouring
// tiles share its L2) and runs its class-0 tiles before its class-1 tiles.
// The class-1 remainder starts at the XCD after the last class-0 remainder,
// so no XCD holds more than ceil((n0 + n1) / 8) tiles.  Needs a grid of at
// least 8 * ceil((n0 + n1) / 8) blocks; returns false for blocks past their
// XCD's tiles.
MOE_DEV bool xcd_slot2(int b, int n0, int n1, int& cls, int& id) {
  const int x = b & 7, j = b >> 3;
  const int q0 = n0 >> 3, r0 = n0 & 7, q1 = n1 >> 3, r1 = n1 & 7;
  const int c0 = q0 + (x < r0 ? 1 : 0);
  if (j < c0) {
    cls = 0;
    id = x * q0 + (x < r0 ? x : r0) + j;
    return true;
  }
  const int xr = (x - r0) & 7;  // rank of this XCD in the class-1 dealing
  const int j1 = j - c0;
  if (j1 >= q1 + (xr < r1 ? 1 : 0)) return false;
  cls = 1;
  id = xr * q1 + (xr < r1 ? xr : r1) + j1;
  return true;
}
