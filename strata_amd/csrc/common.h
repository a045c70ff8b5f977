// Shared helpers for the gfx950 kernels: vector types, bf16 packing, error
// reporting for the C ABI, and NATTEN's clamped-window arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/strata_hip.h"

namespace strata {

typedef __bf16 bf16;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

// ---- error reporting (thread-local message behind strata_hip_last_error) ----
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// ---- bf16 helpers ----------------------------------------------------------
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  // Round-to-nearest-even conversion; gfx950 lowers this to v_cvt_pk_bf16_f32.
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v = {(bf16)a, (bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---- NATTEN window arithmetic ---------------------------------------------
// One axis of length L, odd kernel k, dilation d.  Query i belongs to residue
// class g = i mod d; inside that class (a grid of ceil((L-g)/d) points) the
// window is the length-k run whose start is clamp(i/d - k/2, 0, Lg - k).
__host__ __device__ __forceinline__ int sub_len(int L, int g, int d) { return (L - g + d - 1) / d; }

__host__ __device__ __forceinline__ int win_start(int ig, int Lg, int k) {
  int s = ig - k / 2;
  s = s < 0 ? 0 : s;
  int hi = Lg - k;
  return s > hi ? hi : s;
}

// First and one-past-last sub-grid index (within residue class g) of the real
// query range [o, o+e).
__host__ __device__ __forceinline__ int sub_first(int o, int g, int d) { return o <= g ? 0 : (o - g + d - 1) / d; }
__host__ __device__ __forceinline__ int sub_end(int o, int e, int g, int d) {
  int hi = o + e;
  return hi <= g ? 0 : (hi - g + d - 1) / d;
}

}  // namespace strata
