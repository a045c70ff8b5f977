// Pixel-stage block pieces (this build's reading of physicsnemo's StrataPixel3DBlock with
// use_bilinear_dw_gelu_project_adaln: screamcast/strata_wrappers.py:443,471-477,490-495;
// parameters adaln_bilinear_dw_{conv,proj} per tests/regression_data/pixeldit_...
// param_order.txt:245-256).  The semantic stage's tokens condition every pixel block
// through a spatially varying adaLN:
//
//   c   = GELU_tanh(dwconv3x3(bilinear_up_f(cond)) + b)     [B, Z, Y, X, Cs]
//   mod = c @ W^T + b_proj -> shift1, scale1, gate1, shift2, scale2, gate2   (each C wide)
//   x   = x + gate1 * attn(LN(x) * (1 + scale1) + shift1)
//   x   = x + gate2 * mlp(LN(x) * (1 + scale2) + shift2)
//
// Three bandwidth-bound kernels here (the projection is the library's GEMM):
//   * upsample_dw_gelu_kernel: bilinear upsampling by f in y and x (align_corners =
//     false, as torch's F.interpolate), the 3x3 depthwise convolution of the upsampled
//     map (zero padding), bias and GELU(tanh), fused into one 3x3 filter on the coarse
//     tokens per output position and channel (formed once per thread, which then walks
//     every z); the upsampled map is never written;
//   * layer_norm_modulate_kernel: the non-affine LayerNorm of a row, then
//     * (1 + scale) + shift from two strided views of the modulation tensor;
//   * gated_add_kernel: out = res + gate * y.
#include "common.h"

namespace strata {

// GELU(tanh) = x * sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3), with 2u log2(e) folded
// into one polynomial (the MLP GEMM's form): one exp2 and one reciprocal.
__device__ __forceinline__ float px_gelu_tanh(float x) {
  constexpr float k1 = 2.f * 1.4426950408889634f * 0.7978845608028654f;
  const float t = x * fmaf(k1 * 0.044715f, x * x, k1);
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-t));
}

// Source index pair and weight of one output coordinate of the bilinear upsampling
// (torch's align_corners = false: src = (o + 0.5) / f - 0.5, clamped at 0; 1 / f as a float,
// as torch's own scale).
__device__ __forceinline__ void bilinear_src(int o, float inv_f, int n, int& i0, int& i1, float& w1) {
  float src = ((float)o + 0.5f) * inv_f - 0.5f;
  src = src < 0.f ? 0.f : src;
  i0 = (int)src;
  i0 = i0 > n - 1 ? n - 1 : i0;
  i1 = i0 + (i0 < n - 1 ? 1 : 0);
  w1 = src - (float)i0;
}

struct UpDwParams {
  const bf16* cond;
  bf16* out;
  const bf16* w;  // [9, C]: tap-major
  const bf16* b;  // [C] or null
  int B, Z, Yc, Xc, C, f;
  int cgw, np, nxb;  // a workgroup's channel groups and output columns; workgroups per output row
  int64_t cs[4], os[4];
};

constexpr int UPDW_STAGE = 1024;  // staged 16-byte runs per z slice (4 per thread)

// A workgroup owns cgw groups of 8 channels x np consecutive output columns of one
// output row (b, y), every z; one thread per (column, channel group).  The 3 x 3
// upsampled neighbourhood of output (y, x) draws on at most 3 x 3 coarse tokens (rows
// r0 .. r0 + 2, columns c0 .. c0 + 2): with by[dy][r] the weight of coarse row r0 + r in
// upsampled row y + dy - 1 (zero outside the map: the convolution's padding) and bx
// likewise, the output is sum_rc K[r][c] cond[r][c] with K = by^T (w bx) per channel,
// formed once per thread.  Per z the workgroup stages the coarse runs its windows touch
// (3 rows x the columns from its first column's c0 to its last's c0 + 2, cgw channel
// groups: at f = 4, 16 columns take 7 coarse columns) in LDS, STG loads per thread,
// the next slice's loads issued before the current slice's arithmetic; each thread then
// reads its 9 runs from LDS and does 9 FMAs per channel.  (One thread loading its own 9
// runs from L2 took 9 vector-memory instructions per 16-byte output.)
template <int STG>
__global__ __launch_bounds__(256) void upsample_dw_gelu_kernel(UpDwParams p) {
  __shared__ u32x4 stage[2][UPDW_STAGE];
  const int tid = (int)threadIdx.x;
  int blk = (int)blockIdx.x;
  const int ncgb = (p.C / 8) / p.cgw;
  const int cgb = blk % ncgb;
  blk /= ncgb;
  const int xb = blk % p.nxb;
  blk /= p.nxb;
  const int Y = p.Yc * p.f, X = p.Xc * p.f;
  const int y = blk % Y;
  const int b = blk / Y;
  const int ci = tid % p.cgw, pi = tid / p.cgw;
  const int x0 = xb * p.np;
  const int xl = min(x0 + p.np, X) - 1;  // the workgroup's last column
  const bool live = pi < p.np && x0 + pi <= xl;
  const int x = live ? x0 + pi : xl;
  const int ch = 8 * (cgb * p.cgw + ci);
  const float inv_f = 1.f / (float)p.f;
  auto c0_of = [&](int xx) {
    int i0, i1;
    float w1;
    bilinear_src(max(xx - 1, 0), inv_f, p.Xc, i0, i1, w1);
    return min(i0, max(p.Xc - 3, 0));
  };
  int r0;
  {
    int i0, i1;
    float w1;
    bilinear_src(max(y - 1, 0), inv_f, p.Yc, i0, i1, w1);
    r0 = min(i0, max(p.Yc - 3, 0));
  }
  const int cfirst = c0_of(x0), c0 = c0_of(x);
  const int ncol = c0_of(xl) - cfirst + 3;
  const int nrun = 3 * ncol * p.cgw;  // <= STG * 256 (the host's bound)
  float by[3][3], bx[3][3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
#pragma unroll
    for (int k = 0; k < 3; ++k) by[d][k] = bx[d][k] = 0.f;
    int i0, i1;
    float w1;
    const int yy = y + d - 1, xx = x + d - 1;
    if (yy >= 0 && yy < Y) {  // else the convolution's zero padding
      bilinear_src(yy, inv_f, p.Yc, i0, i1, w1);
#pragma unroll
      for (int k = 0; k < 3; ++k) by[d][k] = (r0 + k == i0 ? 1.f - w1 : 0.f) + (r0 + k == i1 ? w1 : 0.f);  // i1 == i0: 1
    }
    if (xx >= 0 && xx < X) {
      bilinear_src(xx, inv_f, p.Xc, i0, i1, w1);
#pragma unroll
      for (int k = 0; k < 3; ++k) bx[d][k] = (c0 + k == i0 ? 1.f - w1 : 0.f) + (c0 + k == i1 ? w1 : 0.f);
    }
  }
  // K[e][r][c] = sum_dy by[dy][r] sum_dx w_e[dy][dx] bx[dx][c]
  float K[8][9];
  {
    u32x4 wv[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) wv[k] = *(const u32x4*)(p.w + (int64_t)k * p.C + ch);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int w2 = e >> 1;
      auto el = [&](const u32x4& q) { return (e & 1) ? bf16_hi(q[w2]) : bf16_lo(q[w2]); };
      float T[3][3];
#pragma unroll
      for (int dy = 0; dy < 3; ++dy)
#pragma unroll
        for (int c = 0; c < 3; ++c)
          T[dy][c] = el(wv[3 * dy]) * bx[0][c] + el(wv[3 * dy + 1]) * bx[1][c] + el(wv[3 * dy + 2]) * bx[2][c];
#pragma unroll
      for (int rr = 0; rr < 3; ++rr)
#pragma unroll
        for (int c = 0; c < 3; ++c) K[e][3 * rr + c] = by[0][rr] * T[0][c] + by[1][rr] * T[1][c] + by[2][rr] * T[2][c];
    }
  }
  float bias[8];
  {
    u32x4 bv = {0u, 0u, 0u, 0u};
    if (p.b) bv = *(const u32x4*)(p.b + ch);
#pragma unroll
    for (int e = 0; e < 8; ++e) bias[e] = (e & 1) ? bf16_hi(bv[e >> 1]) : bf16_lo(bv[e >> 1]);
  }
  // Staged run s = (row i, column j, group g) at (i * ncol + j) * cgw + g; coarse rows and
  // columns past a grid of fewer than 3 repeat the last (their weights are 0).
  int64_t soff[STG];
#pragma unroll
  for (int u = 0; u < STG; ++u) {
    const int s = min(tid + 256 * u, nrun - 1);
    const int i = s / (ncol * p.cgw), rem = s % (ncol * p.cgw);
    soff[u] = (int64_t)min(r0 + i, p.Yc - 1) * p.cs[2] + (int64_t)min(cfirst + rem / p.cgw, p.Xc - 1) * p.cs[3] +
              8 * (cgb * p.cgw + rem % p.cgw);
  }
  const int tbase = (c0 - cfirst) * p.cgw + ci;  // tap (i, j) at tbase + (i * ncol + j) * cgw
  const bf16* cb = p.cond + (int64_t)b * p.cs[0];
  bf16* ob = p.out + (int64_t)b * p.os[0] + (int64_t)y * p.os[2] + (int64_t)x * p.os[3] + ch;
  u32x4 g[STG];
  auto gload = [&](int z) {
#pragma unroll
    for (int u = 0; u < STG; ++u) g[u] = *(const u32x4*)(cb + (int64_t)z * p.cs[1] + soff[u]);
  };
  auto sput = [&](int buf) {
#pragma unroll
    for (int u = 0; u < STG; ++u)
      if (tid + 256 * u < nrun) stage[buf][tid + 256 * u] = g[u];
  };
  gload(0);
  sput(0);
  __syncthreads();
  for (int z = 0; z < p.Z; ++z) {  // every thread runs every slice (the barriers)
    if (z + 1 < p.Z) gload(z + 1);
    if (live) {
      // tap-major: one staged run live at a time (each channel's sum in the same order)
      float acc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = bias[e];
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        const u32x4 v = stage[z & 1][tbase + ((k / 3) * ncol + k % 3) * p.cgw];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(K[e][k], (e & 1) ? bf16_hi(v[e >> 1]) : bf16_lo(v[e >> 1]), acc[e]);
      }
      u32x4 o;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) o[w2] = pack_bf16x2(px_gelu_tanh(acc[2 * w2]), px_gelu_tanh(acc[2 * w2 + 1]));
      *(u32x4*)(ob + (int64_t)z * p.os[1]) = o;
    }
    if (z + 1 < p.Z) sput((z + 1) & 1);  // the slot read one slice ago (the barrier below orders it)
    __syncthreads();
  }
}

// LPR lanes per row, NR runs of 8 channels per lane (as layer_norm_kernel).
template <int LPR, int NR>
__global__ __launch_bounds__(256) void layer_norm_modulate_kernel(const bf16* __restrict__ x, bf16* __restrict__ out,
                                                                  const bf16* __restrict__ shift,
                                                                  const bf16* __restrict__ scale, int64_t M, int C,
                                                                  int64_t ldx, int64_t ldo, int64_t ldsh, int64_t ldsc,
                                                                  float eps) {
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
  float tot = s;
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) tot += __shfl_xor(tot, o);
  const float mean = tot / C;
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
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) q += __shfl_xor(q, o);
  const float rstd = rsqrtf(q / C + eps);
  const bf16* shr = shift + row * ldsh;
  const bf16* scr = scale + row * ldsc;
  bf16* orow = out + row * ldo;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int run = lane + LPR * r;
    if (run < runs) {
      const u32x4 sh = *(const u32x4*)(shr + 8 * run), sc = *(const u32x4*)(scr + 8 * run);
      u32x4 o;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float lo = (bf16_lo(v[r][w]) - mean) * rstd, hi = (bf16_hi(v[r][w]) - mean) * rstd;
        o[w] = pack_bf16x2(fmaf(lo, 1.f + bf16_lo(sc[w]), bf16_lo(sh[w])), fmaf(hi, 1.f + bf16_hi(sc[w]), bf16_hi(sh[w])));
      }
      *(u32x4*)(orow + 8 * run) = o;
    }
  }
}

__global__ __launch_bounds__(256) void gated_add_kernel(const bf16* __restrict__ res, const bf16* __restrict__ gate,
                                                        const bf16* __restrict__ y, bf16* __restrict__ out, int64_t M,
                                                        int C, int64_t ldr, int64_t ldg, int64_t ldy, int64_t ldo) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int cg = C / 8;
  if (t >= M * cg) return;
  const int64_t m = t / cg;
  const int c = 8 * (int)(t % cg);
  const u32x4 r = *(const u32x4*)(res + m * ldr + c), g = *(const u32x4*)(gate + m * ldg + c),
              v = *(const u32x4*)(y + m * ldy + c);
  u32x4 o;
#pragma unroll
  for (int w = 0; w < 4; ++w)
    o[w] = pack_bf16x2(fmaf(bf16_lo(g[w]), bf16_lo(v[w]), bf16_lo(r[w])),
                       fmaf(bf16_hi(g[w]), bf16_hi(v[w]), bf16_hi(r[w])));
  *(u32x4*)(out + m * ldo + c) = o;
}

static bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace strata

using namespace strata;

extern "C" int strata_hip_upsample_dw_gelu(const strata_hip_upsample_dw_gelu_args* a, void* stream) {
  if (!a || !a->cond || !a->out || !a->weight) return fail(STRATA_HIP_EINVAL, "upsample_dw_gelu: null pointer");
  if (a->batch < 0 || a->depth < 0 || a->height <= 0 || a->width <= 0 || a->channels <= 0 || a->factor <= 0)
    return fail(STRATA_HIP_EINVAL, "upsample_dw_gelu: bad shape or factor");
  if (a->channels % 8 || !al16(a->cond) || !al16(a->out))
    return fail(STRATA_HIP_EINVAL, "upsample_dw_gelu: channels must be a multiple of 8, tensors 16-byte aligned");
  for (int i = 0; i < 4; ++i)
    if (a->cond_stride[i] % 8 || a->out_stride[i] % 8 || a->cond_stride[i] < 0 || a->out_stride[i] < 0)
      return fail(STRATA_HIP_EINVAL, "upsample_dw_gelu: strides must be non-negative multiples of 8 elements");
  UpDwParams p;
  p.cond = (const bf16*)a->cond;
  p.out = (bf16*)a->out;
  p.w = (const bf16*)a->weight;
  p.b = (const bf16*)a->bias;
  p.B = a->batch;
  p.Z = a->depth;
  p.Yc = a->height;
  p.Xc = a->width;
  p.C = a->channels;
  p.f = a->factor;
  for (int i = 0; i < 4; ++i) {
    p.cs[i] = a->cond_stride[i];
    p.os[i] = a->out_stride[i];
  }
  if (p.B == 0 || p.Z == 0) return STRATA_HIP_OK;
  // Channel groups per workgroup: the largest divisor of C / 8 up to 16; the rest of the
  // 256 threads take consecutive output columns.
  const int cg = p.C / 8;
  p.cgw = 1;
  for (int d = 16; d >= 1; --d)
    if (cg % d == 0) {
      p.cgw = d;
      break;
    }
  p.np = 256 / p.cgw;
  const int64_t X = (int64_t)p.Xc * p.f, Y = (int64_t)p.Yc * p.f;
  p.nxb = (int)((X + p.np - 1) / p.np);
  // Staged runs per slice: 3 rows x at most (np - 1) / f + 4 coarse columns (the span of
  // the columns' c0, plus 3) x cgw; with np * cgw <= 256 and cgw <= 16, at most 912.
  const int64_t nrun_max = 3 * ((int64_t)(p.np - 1) / p.f + 4) * p.cgw;
  if (nrun_max > UPDW_STAGE) return fail(STRATA_HIP_EUNSUPPORTED, "upsample_dw_gelu: staging bound");
  const int64_t blocks = (int64_t)p.B * Y * p.nxb * (cg / p.cgw);
  if (blocks > 0x7fffffff || X > 0x7fffffff / 4) return fail(STRATA_HIP_EUNSUPPORTED, "upsample_dw_gelu: too large");
  if (nrun_max <= 512)
    hipLaunchKernelGGL(upsample_dw_gelu_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(upsample_dw_gelu_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
  return check_launch("upsample_dw_gelu_kernel");
}

template <int LPR, int NR>
static void launch_lnm(const strata_hip_layer_norm_modulate_args* a, hipStream_t st) {
  const int64_t rows = 256 / LPR;
  hipLaunchKernelGGL((layer_norm_modulate_kernel<LPR, NR>), dim3((unsigned)((a->m + rows - 1) / rows)), dim3(256), 0,
                     st, (const bf16*)a->x, (bf16*)a->out, (const bf16*)a->shift, (const bf16*)a->scale, a->m,
                     (int)a->c, a->ldx, a->ldo, a->ld_shift, a->ld_scale, a->eps);
}

extern "C" int strata_hip_layer_norm_modulate(const strata_hip_layer_norm_modulate_args* a, void* stream) {
  if (!a || !a->x || !a->out || !a->shift || !a->scale) return fail(STRATA_HIP_EINVAL, "layer_norm_modulate: null pointer");
  if (a->m < 0 || a->c <= 0 || a->c % 8 || a->c > 4096)
    return fail(STRATA_HIP_EINVAL, "layer_norm_modulate: channels must be a positive multiple of 8, at most 4096");
  if (!al16(a->x) || !al16(a->out) || !al16(a->shift) || !al16(a->scale) || a->ldx % 8 || a->ldo % 8 ||
      a->ld_shift % 8 || a->ld_scale % 8)
    return fail(STRATA_HIP_EINVAL, "layer_norm_modulate: tensors 16-byte aligned, row strides multiples of 8");
  if (a->m == 0) return STRATA_HIP_OK;
  if ((a->m + 3) / 4 > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "layer_norm_modulate: too many rows");
  const hipStream_t st = (hipStream_t)stream;
  const int runs = (int)(a->c / 8);
  if (runs <= 16)
    launch_lnm<16, 1>(a, st);
  else if (runs <= 32)
    launch_lnm<32, 1>(a, st);
  else if (runs <= 64)
    launch_lnm<64, 1>(a, st);
  else if (runs <= 128)
    launch_lnm<64, 2>(a, st);
  else if (runs <= 256)
    launch_lnm<64, 4>(a, st);
  else
    launch_lnm<64, 8>(a, st);
  return check_launch("layer_norm_modulate_kernel");
}

extern "C" int strata_hip_gated_add(const strata_hip_gated_add_args* a, void* stream) {
  if (!a || !a->res || !a->gate || !a->y || !a->out) return fail(STRATA_HIP_EINVAL, "gated_add: null pointer");
  if (a->m < 0 || a->c <= 0 || a->c % 8) return fail(STRATA_HIP_EINVAL, "gated_add: channels must be a multiple of 8");
  if (!al16(a->res) || !al16(a->gate) || !al16(a->y) || !al16(a->out) || a->ld_res % 8 || a->ld_gate % 8 ||
      a->ld_y % 8 || a->ld_out % 8)
    return fail(STRATA_HIP_EINVAL, "gated_add: tensors 16-byte aligned, row strides multiples of 8");
  const int64_t total = a->m * (a->c / 8);
  if (total == 0) return STRATA_HIP_OK;
  if ((total + 255) / 256 > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "gated_add: too large");
  hipLaunchKernelGGL(gated_add_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const bf16*)a->res, (const bf16*)a->gate, (const bf16*)a->y, (bf16*)a->out, a->m, (int)a->c,
                     a->ld_res, a->ld_gate, a->ld_y, a->ld_out);
  return check_launch("gated_add_kernel");
}
