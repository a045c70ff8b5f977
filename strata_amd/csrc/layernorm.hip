// Non-affine LayerNorm over the channel dimension, bf16 in/out, fp32 stats.
// One wave per row (or, when a row's 16-byte runs split evenly over 32 lanes
// but not over 64, e.g. 768 channels, half a wave per row); each lane keeps
// its 16-byte runs of the row in registers (rows up to 4096 channels) so the
// row is read from HBM once.
#include "common.h"

namespace strata {

constexpr int LN_MAX_RUNS = 8;  // 8 runs x 8 elements x 64 lanes = 4096 channels

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Sum over the LPR lanes that share a row (aligned groups of LPR lanes).
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// LPR lanes per row (64 or 32): 256 / LPR rows per 256-thread block; NR
// register slots of 16 bytes per lane (at least C / 8 / LPR: the instance is
// picked by the row length, so short rows keep few registers and many waves).
template <int LPR, int NR>
__global__ __launch_bounds__(256) void layer_norm_kernel(const bf16* __restrict__ x, bf16* __restrict__ out, int64_t M,
                                                         int C, int64_t ldx, int64_t ldo, float eps) {
  const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + (threadIdx.x / LPR);
  if (row >= M) return;  // uniform over a row's lanes
  const int lane = threadIdx.x % LPR;
  const int runs = C / 8;
  const bf16* xr = x + row * ldx;
  u32x4 v[NR];
  float s = 0.f;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int run = lane + LPR * r;
    v[r] = (u32x4){0u, 0u, 0u, 0u};
    if (run < runs) {
      v[r] = *(const u32x4*)(xr + 8 * run);
#pragma unroll
      for (int w = 0; w < 4; ++w) s += bf16_lo(v[r][w]) + bf16_hi(v[r][w]);
    }
  }
  const float mean = row_sum<LPR>(s) / C;
  float q = 0.f;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if (lane + LPR * r < runs) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float a = bf16_lo(v[r][w]) - mean, b = bf16_hi(v[r][w]) - mean;
        q = fmaf(a, a, q);
        q = fmaf(b, b, q);
      }
    }
  }
  const float rstd = rsqrtf(row_sum<LPR>(q) / C + eps);
  bf16* orow = out + row * ldo;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int run = lane + LPR * r;
    if (run < runs) {
      u32x4 o;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        o[w] = pack_bf16x2((bf16_lo(v[r][w]) - mean) * rstd, (bf16_hi(v[r][w]) - mean) * rstd);
      *(u32x4*)(orow + 8 * run) = o;
    }
  }
}

// Backward of the non-affine LayerNorm, one wave per row as above:
//   xh = (x - mean) * rstd,  dx = rstd * (dy - mean(dy) - xh * mean(dy * xh)).
// NR register slots of 16 bytes per lane for each of x and dy, as above.
template <int NR>
__global__ __launch_bounds__(256) void layer_norm_bwd_kernel(const bf16* __restrict__ x, const bf16* __restrict__ dy,
                                                             bf16* __restrict__ dx, int64_t M, int C, int64_t ld,
                                                             float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int lane = threadIdx.x & 63;
  const int runs = C / 8;
  u32x4 v[NR], g[NR];
  float s = 0.f;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int run = lane + 64 * r;
    v[r] = g[r] = (u32x4){0u, 0u, 0u, 0u};
    if (run < runs) {
      v[r] = *(const u32x4*)(x + row * ld + 8 * run);
      g[r] = *(const u32x4*)(dy + row * ld + 8 * run);
#pragma unroll
      for (int w = 0; w < 4; ++w) s += bf16_lo(v[r][w]) + bf16_hi(v[r][w]);
    }
  }
  const float mean = wave_sum(s) / C;
  float q = 0.f;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if (lane + 64 * r < runs) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float a = bf16_lo(v[r][w]) - mean, b = bf16_hi(v[r][w]) - mean;
        q = fmaf(a, a, q);
        q = fmaf(b, b, q);
      }
    }
  }
  const float rstd = rsqrtf(wave_sum(q) / C + eps);
  float sg = 0.f, sgx = 0.f;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if (lane + 64 * r < runs) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float g0 = bf16_lo(g[r][w]), g1 = bf16_hi(g[r][w]);
        sg += g0 + g1;
        sgx = fmaf(g0, (bf16_lo(v[r][w]) - mean) * rstd, sgx);
        sgx = fmaf(g1, (bf16_hi(v[r][w]) - mean) * rstd, sgx);
      }
    }
  }
  const float mg = wave_sum(sg) / C, mgx = wave_sum(sgx) / C;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int run = lane + 64 * r;
    if (run < runs) {
      u32x4 o;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float x0 = (bf16_lo(v[r][w]) - mean) * rstd, x1 = (bf16_hi(v[r][w]) - mean) * rstd;
        o[w] = pack_bf16x2(rstd * (bf16_lo(g[r][w]) - mg - x0 * mgx), rstd * (bf16_hi(g[r][w]) - mg - x1 * mgx));
      }
      *(u32x4*)(dx + row * ld + 8 * run) = o;
    }
  }
}

}  // namespace strata

using namespace strata;

extern "C" int strata_hip_layer_norm_bwd(const strata_hip_layer_norm_bwd_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "layer_norm_bwd: null args");
  if (a->m < 0 || a->c <= 0) return fail(STRATA_HIP_EINVAL, "layer_norm_bwd: bad m/c");
  if (a->m == 0) return STRATA_HIP_OK;
  if (!a->x || !a->dy || !a->dx) return fail(STRATA_HIP_EINVAL, "layer_norm_bwd: null pointer");
  if (a->c % 8 || a->c > 8 * 64 * LN_MAX_RUNS)
    return fail(STRATA_HIP_EUNSUPPORTED, "layer_norm_bwd: channels must be a multiple of 8 and at most 4096");
  if (a->ld < a->c || a->ld % 8 || ((uintptr_t)a->x & 15) || ((uintptr_t)a->dy & 15) || ((uintptr_t)a->dx & 15))
    return fail(STRATA_HIP_EINVAL, "layer_norm_bwd: rows must be 16-byte aligned with a stride >= c");
  if (!(a->eps >= 0.f)) return fail(STRATA_HIP_EINVAL, "layer_norm_bwd: eps must be non-negative");
  const int64_t blocks = (a->m + 3) / 4;
  if (blocks > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "layer_norm_bwd: too many rows");
  const int per_lane = (int)((a->c / 8 + 63) / 64);
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (const bf16*)a->x,
                       (const bf16*)a->dy, (bf16*)a->dx, a->m, (int)a->c, a->ld, a->eps);
  };
  if (per_lane <= 2) launch(layer_norm_bwd_kernel<2>);
  else if (per_lane <= 4) launch(layer_norm_bwd_kernel<4>);
  else launch(layer_norm_bwd_kernel<8>);
  return check_launch("layer_norm_bwd_kernel");
}

extern "C" int strata_hip_layer_norm(const strata_hip_layer_norm_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "layer_norm: null args");
  if (a->m < 0 || a->c <= 0) return fail(STRATA_HIP_EINVAL, "layer_norm: bad m/c");
  if (a->m == 0) return STRATA_HIP_OK;
  if (!a->x || !a->out) return fail(STRATA_HIP_EINVAL, "layer_norm: null pointer");
  if (a->c % 8 || a->c > 8 * 64 * LN_MAX_RUNS)
    return fail(STRATA_HIP_EUNSUPPORTED, "layer_norm: channels must be a multiple of 8 and at most 4096");
  if (a->ldx < a->c || a->ldo < a->c || a->ldx % 8 || a->ldo % 8 || ((uintptr_t)a->x & 15) || ((uintptr_t)a->out & 15))
    return fail(STRATA_HIP_EINVAL, "layer_norm: rows must be 16-byte aligned with strides >= c");
  if (!(a->eps >= 0.f)) return fail(STRATA_HIP_EINVAL, "layer_norm: eps must be non-negative");
  // Half a wave per row when the runs fill 32 lanes evenly and 64 lanes would
  // leave half of them idle on the last run (768 channels: 3 runs on 32 lanes
  // instead of 2 on 64, the second half empty).
  const int runs = (int)(a->c / 8);
  const bool half = runs % 64 != 0 && runs % 32 == 0;
  const int rows_per_block = half ? 8 : 4;
  const int64_t blocks = (a->m + rows_per_block - 1) / rows_per_block;
  if (blocks > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "layer_norm: too many rows");
  const int per_lane = (runs + (half ? 32 : 64) - 1) / (half ? 32 : 64);
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (const bf16*)a->x,
                       (bf16*)a->out, a->m, (int)a->c, a->ldx, a->ldo, a->eps);
  };
  if (half) {
    if (per_lane <= 2) launch(layer_norm_kernel<32, 2>);
    else if (per_lane <= 4) launch(layer_norm_kernel<32, 4>);
    else if (per_lane <= 8) launch(layer_norm_kernel<32, 8>);
    else launch(layer_norm_kernel<32, 16>);
  } else {
    if (per_lane <= 2) launch(layer_norm_kernel<64, 2>);
    else if (per_lane <= 4) launch(layer_norm_kernel<64, 4>);
    else launch(layer_norm_kernel<64, 8>);
  }
  return check_launch("layer_norm_kernel");
}
