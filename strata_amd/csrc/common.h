// Shared helpers for the gfx950 kernels: vector types, bf16 packing, error
// reporting for the C ABI, and NATTEN's clamped-window arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <utility>

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

// ---- rotary embedding of one channel pair (a, b) by angle (cos c, sin s) ----
// a' = a c - b s and b' = a s + b c with the fused multiply-adds written out, so
// every kernel that rotates (the RoPE pack, the query rotation inside NA3D, the
// qkv GEMM's RoPE epilogue) rounds alike and their outputs agree bit for bit.
__device__ __forceinline__ float rope_rot_a(float a, float b, float c, float s) { return fmaf(a, c, -(b * s)); }
__device__ __forceinline__ float rope_rot_b(float a, float b, float c, float s) { return fmaf(a, s, b * c); }

// ---- global -> LDS streaming (buffer_load ... lds) ------------------------
constexpr uint32_t OOB = 0x7ffffff0u;  // lane offset / record count that reads as zero

__device__ __forceinline__ void wait_vmcnt(int n) {
  // gfx9 s_waitcnt immediate: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]
  switch (n) {
#define STRATA_VMCNT(N) \
  case N:               \
    __builtin_amdgcn_s_waitcnt(((N) & 15) | (7 << 4) | (15 << 8) | (((N) >> 4) << 14)); \
    break;
    STRATA_VMCNT(0) STRATA_VMCNT(1) STRATA_VMCNT(2) STRATA_VMCNT(3) STRATA_VMCNT(4) STRATA_VMCNT(5)
    STRATA_VMCNT(6) STRATA_VMCNT(7) STRATA_VMCNT(8) STRATA_VMCNT(9) STRATA_VMCNT(10) STRATA_VMCNT(11)
    STRATA_VMCNT(12) STRATA_VMCNT(13) STRATA_VMCNT(14) STRATA_VMCNT(15) STRATA_VMCNT(16)
    STRATA_VMCNT(24) STRATA_VMCNT(32)
#undef STRATA_VMCNT
    default:
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
  }
}

__device__ __forceinline__ void wait_lgkm0() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14));  // lgkmcnt(0), vmcnt/expcnt untouched
}

// One 1-KiB global->LDS copy: lane i's 16 bytes at `voff` within the buffer
// described by `rsrc` land at LDS byte address `lds_addr + 16*i`; offsets
// beyond the descriptor's record count read as zero.  Issued as inline asm so
// that the compiler does not add its own conservative vmcnt(0) before every
// later LDS read (it cannot tell the ring slots apart); completion is tracked
// explicitly with wait_vmcnt() before the barrier that publishes a stage.
__device__ __forceinline__ void dma_row16(u32x4 rsrc, uint32_t lds_addr, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds_addr),
      "v"(voff), "s"(rsrc)
      : "memory", "m0");
}

// One dword per lane into LDS at lds_addr + 4 * lane (as dma_row16).
__device__ __forceinline__ void dma_dword(u32x4 rsrc, uint32_t lds_addr, uint32_t voff) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %1, %2, 0 offen lds" ::"s"(lds_addr),
      "v"(voff), "s"(rsrc)
      : "memory", "m0");
}

__device__ __forceinline__ u32x4 make_rsrc(const void* base, uint32_t num_records) {
  const uint64_t a = (uint64_t)base;
  // dword1 holds base[47:32] with stride 0; dword3 = gfx9 data/num format for raw buffers.
  // Every operand is workgroup-uniform; readfirstlane pins the descriptor in SGPRs.
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  const uint32_t nr = (uint32_t)__builtin_amdgcn_readfirstlane((int)num_records);
  return (u32x4){lo, hi, nr, 0x00020000u};
}

// Workgroup barrier without the release/acquire fences of __syncthreads():
// those would also wait for the in-flight global->LDS loads of later stages.
// LDS visibility is established by each wave's own vmcnt wait before it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

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

// ---- launch order and compile-time loops --------------------------------
// Linear workgroup id remapped so that consecutive tiles run on one XCD:
// the dispatcher deals workgroups round-robin over the 8 XCDs, so XCD k gets
// ids k, k+8, ...; map those to the k-th contiguous block of tiles.
// (__builtin_amdgcn_workgroup_id_x keeps the id visibly uniform to the
// compiler, unlike blockIdx.x's out-of-line library call.)
__device__ __forceinline__ int xcd_tile_order(int n, int id) {
  const int xcd = id & 7, local = id >> 3;
  const int q = n >> 3, rem = n & 7;
  return xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
}

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace strata
