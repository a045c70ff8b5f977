// bf16 GEMM with a fused epilogue for gfx950:  out = act(x @ w^T + bias) + residual
//
// x is [M, K] (activations, K contiguous) and w is [N, K] (nn.Linear weight,
// K contiguous), so both MFMA operands read K-contiguous 16-byte runs.  The
// kernel computes C^T tiles: the weight tile is the MFMA A operand (MFMA rows
// = output columns n) and the activation tile the B operand (MFMA columns =
// output rows m).  A lane of v_mfma_f32_32x32x16_bf16 then owns 4 consecutive
// output columns of one row per accumulator quad, which the epilogue stores
// as one 8-byte write after bias, GELU and residual.
//
// Workgroup tile BM x BN (rows of x x rows of w), K step 64, four waves in a
// 2 x 2 arrangement, LDS double buffer filled from registers one K step ahead.
#include "common.h"

namespace strata {

struct GemmParams {
  const bf16* x;
  const bf16* w;
  const bf16* bias;
  const bf16* res;
  bf16* out;
  int64_t M, N, K;
  int64_t ldx, ldw, ldr, ldo;
  int act;
  int mt, nt;  // tiles along M and N
};

__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
  const float u = 0.7978845608028654f * fmaf(0.044715f * x * x, x, x);
  return 0.5f * x * (1.f + tanhf(u));
}
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.7071067811865476f)); }

template <int BM, int BN, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_bias_act_kernel(GemmParams p) {
  constexpr int BK = 64;
  constexpr int NT = 64 * WGM * WGN;
  constexpr int WTM = BM / WGM;  // wave tile along m (MFMA N)
  constexpr int WTN = BN / WGN;  // wave tile along n (MFMA M)
  constexpr int FM = WTM / 32;
  constexpr int FN = WTN / 32;
  constexpr int XCH = BM * BK / 8;  // 16-byte chunks per x tile
  constexpr int WCH = BN * BK / 8;
  constexpr int XCPT = (XCH + NT - 1) / NT;
  constexpr int WCPT = (WCH + NT - 1) / NT;
  constexpr int STAGE = (BM + BN) * BK;

  __shared__ __attribute__((aligned(16))) bf16 lds[2 * STAGE];

  int wg;
  {
    const int id = blockIdx.x, n = gridDim.x;
    const int xcd = id & 7, local = id >> 3;
    const int q = n >> 3, rem = n & 7;
    wg = xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
  }
  const int tn = wg % p.nt;
  const int tm = wg / p.nt;
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * BN;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int wm = wave / WGN;
  const int wn = wave % WGN;
  const int l32 = lane & 31;
  const int hi = lane >> 5;

  u32x4 xr[XCPT], wr[WCPT];
  auto load_tile = [&](int64_t k0) {
#pragma unroll
    for (int c = 0; c < XCPT; ++c) {
      const int ci = tid + c * NT;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (ci < XCH) {
        const int row = ci >> 3, ch = ci & 7;
        const int64_t gm = m0 + row, gk = k0 + 8 * ch;
        if (gm < p.M && gk < p.K) v = *(const u32x4*)(p.x + gm * p.ldx + gk);
      }
      xr[c] = v;
    }
#pragma unroll
    for (int c = 0; c < WCPT; ++c) {
      const int ci = tid + c * NT;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (ci < WCH) {
        const int row = ci >> 3, ch = ci & 7;
        const int64_t gn = n0 + row, gk = k0 + 8 * ch;
        if (gn < p.N && gk < p.K) v = *(const u32x4*)(p.w + gn * p.ldw + gk);
      }
      wr[c] = v;
    }
  };
  auto store_tile = [&](int buf) {
    bf16* xs = lds + buf * STAGE;
    bf16* ws = xs + BM * BK;
#pragma unroll
    for (int c = 0; c < XCPT; ++c) {
      const int ci = tid + c * NT;
      if (ci < XCH) {
        const int row = ci >> 3, ch = ci & 7;
        *(u32x4*)(xs + row * BK + 8 * (ch ^ (row & 7))) = xr[c];
      }
    }
#pragma unroll
    for (int c = 0; c < WCPT; ++c) {
      const int ci = tid + c * NT;
      if (ci < WCH) {
        const int row = ci >> 3, ch = ci & 7;
        *(u32x4*)(ws + row * BK + 8 * (ch ^ (row & 7))) = wr[c];
      }
    }
  };

  f32x16 acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = (int)((p.K + BK - 1) / BK);
  load_tile(0);
  store_tile(0);
  for (int kt = 0; kt < nk; ++kt) {
    __syncthreads();
    if (kt + 1 < nk) load_tile((int64_t)(kt + 1) * BK);
    const bf16* xs = lds + (kt & 1) * STAGE;
    const bf16* ws = xs + BM * BK;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int ch = 2 * kk + hi;
      bf16x8 af[FN], bfr[FM];
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const int row = wn * WTN + 32 * i + l32;
        af[i] = *(const bf16x8*)(ws + row * BK + 8 * (ch ^ (row & 7)));
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int row = wm * WTM + 32 * j + l32;
        bfr[j] = *(const bf16x8*)(xs + row * BK + 8 * (ch ^ (row & 7)));
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_tile((kt + 1) & 1);
  }

  // ---- epilogue: lane owns row m, columns n .. n+3 of each quad ----
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int64_t gm = m0 + wm * WTM + 32 * j + l32;
    if (gm >= p.M) continue;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t gn = n0 + wn * WTN + 32 * i + 8 * q + 4 * hi;
        if (gn >= p.N) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e];
        const bool full = gn + 4 <= p.N;
        if (p.bias) {
          if (full) {
            const u32x2 bw = *(const u32x2*)(p.bias + gn);
            v[0] += bf16_lo(bw[0]);
            v[1] += bf16_hi(bw[0]);
            v[2] += bf16_lo(bw[1]);
            v[3] += bf16_hi(bw[1]);
          } else {
            for (int e = 0; e < 4 && gn + e < p.N; ++e) v[e] += (float)p.bias[gn + e];
          }
        }
        if (p.act == STRATA_HIP_ACT_GELU_TANH) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(v[e]);
        } else if (p.act == STRATA_HIP_ACT_GELU_ERF) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = gelu_erf(v[e]);
        }
        if (full) {
          if (p.res) {
            const u32x2 rw = *(const u32x2*)(p.res + gm * p.ldr + gn);
            v[0] += bf16_lo(rw[0]);
            v[1] += bf16_hi(rw[0]);
            v[2] += bf16_lo(rw[1]);
            v[3] += bf16_hi(rw[1]);
          }
          const u32x2 ow = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
          *(u32x2*)(p.out + gm * p.ldo + gn) = ow;
        } else {
          for (int e = 0; e < 4 && gn + e < p.N; ++e) {
            float o = v[e];
            if (p.res) o += (float)p.res[gm * p.ldr + gn + e];
            p.out[gm * p.ldo + gn + e] = (bf16)o;
          }
        }
      }
    }
  }
}

template <int BM, int BN, int WGM, int WGN>
static int launch_gemm(GemmParams p, hipStream_t st) {
  p.mt = (int)((p.M + BM - 1) / BM);
  p.nt = (int)((p.N + BN - 1) / BN);
  const int64_t total = (int64_t)p.mt * p.nt;
  if (total > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "gemm: problem too large for one launch");
  hipLaunchKernelGGL((gemm_bias_act_kernel<BM, BN, WGM, WGN>), dim3((unsigned)total), dim3(64 * WGM * WGN), 0, st, p);
  return check_launch("gemm_bias_act_kernel");
}

}  // namespace strata

using namespace strata;

extern "C" int strata_hip_gemm_bias_act(const strata_hip_gemm_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "gemm: null args");
  if (a->m < 0 || a->n < 0 || a->k <= 0) return fail(STRATA_HIP_EINVAL, "gemm: bad m/n/k");
  if (a->m == 0 || a->n == 0) return STRATA_HIP_OK;
  if (!a->x || !a->w || !a->out) return fail(STRATA_HIP_EINVAL, "gemm: null x, w or out");
  if (a->k % 8 != 0) return fail(STRATA_HIP_EINVAL, "gemm: k must be a multiple of 8");
  if (a->ldx < a->k || a->ldw < a->k || a->ldo < a->n || (a->residual && a->ldr < a->n))
    return fail(STRATA_HIP_EINVAL, "gemm: row stride smaller than the row length");
  if (a->ldx % 8 || a->ldw % 8 || a->ldo % 4 || (a->residual && a->ldr % 4))
    return fail(STRATA_HIP_EINVAL, "gemm: x/w row strides must be multiples of 8, out/residual of 4");
  if (((uintptr_t)a->x & 15) || ((uintptr_t)a->w & 15) || ((uintptr_t)a->out & 7) ||
      (a->residual && ((uintptr_t)a->residual & 7)) || (a->bias && ((uintptr_t)a->bias & 7)))
    return fail(STRATA_HIP_EINVAL, "gemm: x/w must be 16-byte aligned, out/residual/bias 8-byte aligned");
  if (a->act < STRATA_HIP_ACT_NONE || a->act > STRATA_HIP_ACT_GELU_ERF) return fail(STRATA_HIP_EINVAL, "gemm: bad act");
  GemmParams p;
  p.x = (const bf16*)a->x;
  p.w = (const bf16*)a->w;
  p.bias = (const bf16*)a->bias;
  p.res = (const bf16*)a->residual;
  p.out = (bf16*)a->out;
  p.M = a->m;
  p.N = a->n;
  p.K = a->k;
  p.ldx = a->ldx;
  p.ldw = a->ldw;
  p.ldr = a->ldr;
  p.ldo = a->ldo;
  p.act = a->act;
  return launch_gemm<128, 128, 2, 2>(p, (hipStream_t)stream);
}
