// Stereographic-RoPE + QKV pack for gfx950 (bandwidth-bound).
//
// Reads the attn.qkv GEMM output [M, (3, H, D)] and the per-token cos/sin
// tables, rotates the channel pairs of q and k, copies v, and writes three
// heads-last [M, H, D] tensors.  Each thread handles one 16-byte run of
// pairs of one (token, head): 8 pairs for the half layout (two 16-byte runs
// D/2 apart), 4 pairs for the interleaved layout (one 16-byte run).  With
// qk_norm, q and k of each (token, head) are RMS-normalised over D first: the
// D/16 (or D/8) threads of a head are consecutive lanes and reduce their sums
// of squares with lane shuffles; the values stay fp32 until after the
// rotation.
#include "common.h"

namespace strata {

struct RopeParams {
  const bf16* qkv;
  const float* cos;
  const float* sin;
  bf16* q;
  bf16* k;
  bf16* v;
  int64_t M;
  int Z, Y, X, Zt, H, D;
  int64_t ld;
  int qk_norm;
  float eps;
  const bf16* qw;  // RMSNorm weights [D] or null
  const bf16* kw;
  // backward with qk_norm only
  const bf16* x;   // the forward's input qkv
  int64_t ldx;
  float* dqw;      // fp32 [D] weight-gradient accumulators or null
  float* dkw;
};

__device__ __forceinline__ void unpack8(const u32x4& a, float* f) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    f[2 * w] = bf16_lo(a[w]);
    f[2 * w + 1] = bf16_hi(a[w]);
  }
}

// RMS-normalise the n values f[] a lane holds of one head; `lanes`
// consecutive lanes (a power of two) hold the head's D values.  dof[i] is the
// channel of f[i] for the weight.
template <int NV>
__device__ __forceinline__ void rms_norm(float* f, const int* dof, int lanes, int D, float eps, const bf16* w) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) ss = fmaf(f[i], f[i], ss);
  for (int o = 1; o < lanes; o <<= 1) ss += __shfl_xor(ss, o);
  const float r = rsqrtf(ss / (float)D + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) f[i] *= w ? r * (float)w[dof[i]] : r;
}

__device__ __forceinline__ int64_t table_row(const RopeParams& p, int64_t tok) {
  const int64_t x = tok % p.X;
  int64_t r = tok / p.X;
  const int64_t y = r % p.Y;
  r /= p.Y;
  const int64_t z = r % p.Z;
  const int64_t b = r / p.Z;
  const int64_t zt = p.Zt == 1 ? 0 : z;
  return ((b * p.Zt + zt) * p.Y + y) * p.X + x;
}

// Rotate 8 half-layout pairs (a[j], b[j]) = (d, d + D/2) and pack to bf16.
__device__ __forceinline__ void rot8(const float* a, const float* b, const float* c, const float* s, u32x4& oa,
                                     u32x4& ob) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float a0 = a[2 * w], a1 = a[2 * w + 1], b0 = b[2 * w], b1 = b[2 * w + 1];
    const float c0 = c[2 * w], c1 = c[2 * w + 1], s0 = s[2 * w], s1 = s[2 * w + 1];
    oa[w] = pack_bf16x2(rope_rot_a(a0, b0, c0, s0), rope_rot_a(a1, b1, c1, s1));
    ob[w] = pack_bf16x2(rope_rot_b(a0, b0, c0, s0), rope_rot_b(a1, b1, c1, s1));
  }
}

// One head's q or k run of the half layout (already loaded: lo = d in [8c, 8c + 8),
// hi = the same + D/2): optional RMSNorm, then rotation.
__device__ __forceinline__ void half_run(const RopeParams& p, const u32x4& lo, const u32x4& hi, bf16* dst,
                                         const float* cs, const float* sn, int c, int cph, const bf16* w) {
  const int half = p.D / 2;
  float f[16];  // f[0..7]: d = 8c + j, f[8..15]: d = 8c + j + D/2
  unpack8(lo, f);
  unpack8(hi, f + 8);
  if (p.qk_norm) {
    int dof[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      dof[j] = 8 * c + j;
      dof[8 + j] = 8 * c + j + half;
    }
    rms_norm<16>(f, dof, cph, p.D, p.eps, w);
  }
  u32x4 oa, ob;
  rot8(f, f + 8, cs, sn, oa, ob);
  *(u32x4*)(dst) = oa;
  *(u32x4*)(dst + half) = ob;
}

// Half layout: pair p = (d = p, d = p + D/2).  A thread takes ROPE_R runs,
// `slice` apart, and issues all their loads before any math (the pass is
// latency-bound: one run per thread leaves too few bytes in flight).  slice
// is a multiple of 64, so the D/16 lanes of a head share one validity and
// their qk_norm shuffles stay within live lanes.
constexpr int ROPE_R = 2;

__global__ __launch_bounds__(256) void rope_pack_half_kernel(RopeParams p, int64_t total, int64_t slice) {
  const int64_t idx0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx0 >= slice) return;
  const int cph = p.D / 16;
  const int half = p.D / 2;
  const int64_t C = (int64_t)p.H * p.D;
  u32x4 raw[ROPE_R][6];
  float cs[ROPE_R][8], sn[ROPE_R][8];
  int64_t dst[ROPE_R];
  int cc[ROPE_R];
  bool ok[ROPE_R];
#pragma unroll
  for (int r = 0; r < ROPE_R; ++r) {
    const int64_t idx = idx0 + r * slice;
    ok[r] = idx < total;
    const int64_t i = ok[r] ? idx : total - 1;  // a dead run reads a live one and stores nothing
    const int c = (int)(i % cph);
    const int64_t th = i / cph;
    const int h = (int)(th % p.H);
    const int64_t tok = th / p.H;
    const bf16* src = p.qkv + tok * p.ld + (int64_t)h * p.D + 8 * c;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (t == 0 && !p.q) continue;  // uniform: k only (the queries are rotated inside NA3D)
      raw[r][2 * t] = *(const u32x4*)(src + t * C);
      raw[r][2 * t + 1] = *(const u32x4*)(src + t * C + half);
    }
    if (p.v) {  // uniform: v is copied only when asked for
      raw[r][4] = *(const u32x4*)(src + 2 * C);
      raw[r][5] = *(const u32x4*)(src + 2 * C + half);
    }
    const int64_t trow = table_row(p, tok) * half + 8 * c;
    *(f32x4*)&cs[r][0] = *(const f32x4*)(p.cos + trow);
    *(f32x4*)&cs[r][4] = *(const f32x4*)(p.cos + trow + 4);
    *(f32x4*)&sn[r][0] = *(const f32x4*)(p.sin + trow);
    *(f32x4*)&sn[r][4] = *(const f32x4*)(p.sin + trow + 4);
    dst[r] = tok * C + (int64_t)h * p.D + 8 * c;
    cc[r] = c;
  }
#pragma unroll
  for (int r = 0; r < ROPE_R; ++r) {
    if (!ok[r]) continue;  // uniform over the lanes of a head
    if (p.q) half_run(p, raw[r][0], raw[r][1], p.q + dst[r], cs[r], sn[r], cc[r], cph, p.qw);
    half_run(p, raw[r][2], raw[r][3], p.k + dst[r], cs[r], sn[r], cc[r], cph, p.kw);
    if (p.v) {
      *(u32x4*)(p.v + dst[r]) = raw[r][4];
      *(u32x4*)(p.v + dst[r] + half) = raw[r][5];
    }
  }
}

// Interleaved layout: pair p = (d = 2p, d = 2p + 1).
// One head's 8 consecutive q or k values (4 pairs): optional RMSNorm, rotation.
__device__ __forceinline__ u32x4 rot_inter(const RopeParams& p, const u32x4& a, const float* c, const float* s, int cc,
                                           int cph, const bf16* w) {
  float f[8];
  unpack8(a, f);
  if (p.qk_norm) {
    int dof[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) dof[j] = 8 * cc + j;
    rms_norm<8>(f, dof, cph, p.D, p.eps, w);
  }
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float x0 = f[2 * k], x1 = f[2 * k + 1];
    o[k] = pack_bf16x2(rope_rot_a(x0, x1, c[k], s[k]), rope_rot_b(x0, x1, c[k], s[k]));
  }
  return o;
}

__global__ __launch_bounds__(256) void rope_pack_inter_kernel(RopeParams p, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int cph = p.D / 8;
  const int c = (int)(idx % cph);
  const int64_t th = idx / cph;
  const int h = (int)(th % p.H);
  const int64_t tok = th / p.H;
  const int half = p.D / 2;
  const int64_t C = (int64_t)p.H * p.D;

  const bf16* src = p.qkv + tok * p.ld + (int64_t)h * p.D + 8 * c;
  const int64_t trow = table_row(p, tok) * half + 4 * c;
  float cs[4], sn[4];
  *(f32x4*)&cs[0] = *(const f32x4*)(p.cos + trow);
  *(f32x4*)&sn[0] = *(const f32x4*)(p.sin + trow);
  const int64_t dst = tok * C + (int64_t)h * p.D + 8 * c;
  if (p.q) *(u32x4*)(p.q + dst) = rot_inter(p, *(const u32x4*)(src), cs, sn, c, cph, p.qw);  // uniform
  *(u32x4*)(p.k + dst) = rot_inter(p, *(const u32x4*)(src + C), cs, sn, c, cph, p.kw);
  if (p.v) *(u32x4*)(p.v + dst) = *(const u32x4*)(src + 2 * C);
}

// Backward of the pack without qk_norm: the gradient of a rotation by theta is
// the rotation by -theta, so d(qkv) gets R(-theta) dq, R(-theta) dk and dv,
// written back into the [M, (3, H, D)] layout of the qkv GEMM's output (the
// row stride p.ld; p.qkv is the destination here, p.q / p.k / p.v the sources).
__global__ __launch_bounds__(256) void rope_unpack_half_kernel(RopeParams p, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int cph = p.D / 16;
  const int c = (int)(idx % cph);
  const int64_t th = idx / cph;
  const int h = (int)(th % p.H);
  const int64_t tok = th / p.H;
  const int half = p.D / 2;
  const int64_t C = (int64_t)p.H * p.D;
  bf16* dst = const_cast<bf16*>(p.qkv) + tok * p.ld + (int64_t)h * p.D + 8 * c;
  const int64_t trow = table_row(p, tok) * half + 8 * c;
  float cs[8], sn[8];
  *(f32x4*)&cs[0] = *(const f32x4*)(p.cos + trow);
  *(f32x4*)&cs[4] = *(const f32x4*)(p.cos + trow + 4);
  *(f32x4*)&sn[0] = *(const f32x4*)(p.sin + trow);
  *(f32x4*)&sn[4] = *(const f32x4*)(p.sin + trow + 4);
#pragma unroll
  for (int i = 0; i < 8; ++i) sn[i] = -sn[i];
  const int64_t src = tok * C + (int64_t)h * p.D + 8 * c;
  const bf16* srcs[2] = {p.q, p.k};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float f[16];
    unpack8(*(const u32x4*)(srcs[t] + src), f);
    unpack8(*(const u32x4*)(srcs[t] + src + half), f + 8);
    u32x4 oa, ob;
    rot8(f, f + 8, cs, sn, oa, ob);
    *(u32x4*)(dst + t * C) = oa;
    *(u32x4*)(dst + t * C + half) = ob;
  }
  *(u32x4*)(dst + 2 * C) = p.v ? *(const u32x4*)(p.v + src) : (u32x4){0u, 0u, 0u, 0u};  // no dv: v's columns are zero
  *(u32x4*)(dst + 2 * C + half) = p.v ? *(const u32x4*)(p.v + src + half) : (u32x4){0u, 0u, 0u, 0u};
}

__global__ __launch_bounds__(256) void rope_unpack_inter_kernel(RopeParams p, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int cph = p.D / 8;
  const int c = (int)(idx % cph);
  const int64_t th = idx / cph;
  const int h = (int)(th % p.H);
  const int64_t tok = th / p.H;
  const int half = p.D / 2;
  const int64_t C = (int64_t)p.H * p.D;
  bf16* dst = const_cast<bf16*>(p.qkv) + tok * p.ld + (int64_t)h * p.D + 8 * c;
  const int64_t trow = table_row(p, tok) * half + 4 * c;
  float cs[4], sn[4];
  *(f32x4*)&cs[0] = *(const f32x4*)(p.cos + trow);
  *(f32x4*)&sn[0] = *(const f32x4*)(p.sin + trow);
  const int64_t src = tok * C + (int64_t)h * p.D + 8 * c;
  const bf16* srcs[2] = {p.q, p.k};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float f[8];
    unpack8(*(const u32x4*)(srcs[t] + src), f);
    u32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float y0 = f[2 * k], y1 = f[2 * k + 1];
      o[k] = pack_bf16x2(y0 * cs[k] + y1 * sn[k], y1 * cs[k] - y0 * sn[k]);
    }
    *(u32x4*)(dst + t * C) = o;
  }
  *(u32x4*)(dst + 2 * C) = p.v ? *(const u32x4*)(p.v + src) : (u32x4){0u, 0u, 0u, 0u};
}

// Backward with qk_norm: each of q and k goes back through the rotation,
// dy = R(-theta) dout, and then through the RMSNorm y = x * r * w with
// r = 1/sqrt(mean(x^2) + eps) recomputed from the forward's input:
//   dx = r * g - x * r^3 * <g, x> / D,  g = dy * w,
// and the weight gradient sums dy * x * r over tokens and heads.  A thread
// holds 16 (half layout) or 8 (interleaved) values of one (token, head); the
// head's D/16 or D/8 threads are consecutive lanes that reduce <x, x> and
// <g, x> with shuffles, as the forward reduces <x, x>.  The grid-stride loop's
// stride is a multiple of the threads per head, so a thread keeps the same
// channels throughout and sums its weight-gradient terms in registers; at the
// end the block adds them per channel in LDS and adds those to the fp32 [D]
// accumulators with one global atomic per channel and block.
template <bool HALF>
__global__ __launch_bounds__(256) void rope_unpack_norm_kernel(RopeParams p, int64_t total) {
  constexpr int NV = HALF ? 16 : 8;
  __shared__ float red[2][1024];
  const int D = p.D;
  const int cph = HALF ? D / 16 : D / 8;
  const int half = D / 2;
  const int64_t C = (int64_t)p.H * D;
  for (int i = threadIdx.x; i < 2 * D; i += blockDim.x) red[i / D][i % D] = 0.f;

  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int c = (int)(idx % cph);
  int dof[NV];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    dof[j] = 8 * c + j;
    if constexpr (HALF) dof[8 + j] = 8 * c + j + half;
  }
  float wv[2][NV], dw[2][NV];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const bf16* w = t ? p.kw : p.qw;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      wv[t][i] = w ? (float)w[dof[i]] : 1.f;
      dw[t][i] = 0.f;
    }
  }
  const bf16* srcs[2] = {p.q, p.k};

  for (; idx < total; idx += stride) {
    const int64_t th = idx / cph;
    const int h = (int)(th % p.H);
    const int64_t tok = th / p.H;
    const bf16* xin = p.x + tok * p.ldx + (int64_t)h * D + 8 * c;
    bf16* dst = const_cast<bf16*>(p.qkv) + tok * p.ld + (int64_t)h * D + 8 * c;
    const int64_t src = tok * C + (int64_t)h * D + 8 * c;
    constexpr int NP = NV / 2;  // rotation pairs of the thread
    float cs[NP], sn[NP];
    const int64_t trow = table_row(p, tok) * half + NP * c;
#pragma unroll
    for (int i = 0; i < NP; i += 4) {
      *(f32x4*)&cs[i] = *(const f32x4*)(p.cos + trow + i);
      *(f32x4*)&sn[i] = *(const f32x4*)(p.sin + trow + i);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float x[NV], o[NV], dy[NV];
      unpack8(*(const u32x4*)(xin + t * C), x);
      unpack8(*(const u32x4*)(srcs[t] + src), o);
      if constexpr (HALF) {
        unpack8(*(const u32x4*)(xin + t * C + half), x + 8);
        unpack8(*(const u32x4*)(srcs[t] + src + half), o + 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) {  // pair (j, 8 + j) = (d, d + D/2)
          dy[j] = o[j] * cs[j] + o[8 + j] * sn[j];
          dy[8 + j] = o[8 + j] * cs[j] - o[j] * sn[j];
        }
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {  // pair (2k, 2k + 1)
          dy[2 * k] = o[2 * k] * cs[k] + o[2 * k + 1] * sn[k];
          dy[2 * k + 1] = o[2 * k + 1] * cs[k] - o[2 * k] * sn[k];
        }
      }
      float ss = 0.f, gx = 0.f, g[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        ss = fmaf(x[i], x[i], ss);
        g[i] = dy[i] * wv[t][i];
        gx = fmaf(g[i], x[i], gx);
      }
      for (int o2 = 1; o2 < cph; o2 <<= 1) {
        ss += __shfl_xor(ss, o2);
        gx += __shfl_xor(gx, o2);
      }
      const float r = rsqrtf(ss / (float)D + p.eps);
      const float coef = r * r * r * gx / (float)D;
      float dx[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        dx[i] = r * g[i] - x[i] * coef;
        dw[t][i] = fmaf(dy[i] * x[i], r, dw[t][i]);
      }
      u32x4 lo, hi;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        lo[w] = pack_bf16x2(dx[2 * w], dx[2 * w + 1]);
        if constexpr (HALF) hi[w] = pack_bf16x2(dx[8 + 2 * w], dx[8 + 2 * w + 1]);
      }
      *(u32x4*)(dst + t * C) = lo;
      if constexpr (HALF) *(u32x4*)(dst + t * C + half) = hi;
    }
    *(u32x4*)(dst + 2 * C) = p.v ? *(const u32x4*)(p.v + src) : (u32x4){0u, 0u, 0u, 0u};
    if constexpr (HALF) *(u32x4*)(dst + 2 * C + half) = p.v ? *(const u32x4*)(p.v + src + half) : (u32x4){0u, 0u, 0u, 0u};
  }

  if (!p.dqw && !p.dkw) return;  // uniform: no weight gradients wanted
  __syncthreads();
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < NV; ++i) atomicAdd(&red[t][dof[i]], dw[t][i]);
  __syncthreads();
  for (int i = threadIdx.x; i < 2 * D; i += blockDim.x) {
    float* acc = i < D ? p.dqw : p.dkw;
    if (acc) unsafeAtomicAdd(acc + i % D, red[i / D][i % D]);
  }
}

}  // namespace strata

using namespace strata;

extern "C" int strata_hip_rope_qkv_pack_bwd(const strata_hip_rope_pack_bwd_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: null args");
  if (!a->dq || !a->dk || !a->cos || !a->sin || !a->dqkv)
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: null pointer");
  if (a->batch < 0 || a->grid[0] <= 0 || a->grid[1] <= 0 || a->grid[2] <= 0 || a->heads <= 0)
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: bad batch/grid/heads");
  if (a->table_z != 1 && a->table_z != a->grid[0])
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: table_z must be 1 or Z");
  if (a->layout != STRATA_HIP_ROPE_HALF && a->layout != STRATA_HIP_ROPE_INTERLEAVED)
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: bad layout");
  if (a->layout == STRATA_HIP_ROPE_HALF ? (a->head_dim % 16) : (a->head_dim % 8))
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: head_dim must be a multiple of 16 (half) or 8 (interleaved)");
  const int64_t C = (int64_t)a->heads * a->head_dim;
  if (a->dqkv_row_stride < 3 * C || a->dqkv_row_stride % 8)
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: dqkv row stride must be >= 3*H*D and a multiple of 8");
  const void* ptrs[6] = {a->dq, a->dk, a->dv, a->cos, a->sin, a->dqkv};
  for (int i = 0; i < 6; ++i)
    if ((uintptr_t)ptrs[i] & 15) return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: pointers must be 16-byte aligned");
  if (a->qk_norm != 0 && a->qk_norm != 1) return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: qk_norm must be 0 or 1");
  if (a->qk_norm) {
    const int cph = a->layout == STRATA_HIP_ROPE_HALF ? a->head_dim / 16 : a->head_dim / 8;
    if (cph < 1 || cph > 64 || (cph & (cph - 1)))
      return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: qk_norm needs D/16 (half) or D/8 (interleaved) a power of two <= 64");
    if (!(a->qk_norm_eps >= 0.f)) return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: qk_norm_eps must be >= 0");
    if (!a->qkv || ((uintptr_t)a->qkv & 15))
      return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: qk_norm needs the forward's qkv, 16-byte aligned");
    if (a->qkv_row_stride < 3 * C || a->qkv_row_stride % 8)
      return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: qkv row stride must be >= 3*H*D and a multiple of 8");
    if (!a->q_norm_weight != !a->dq_norm_weight || !a->k_norm_weight != !a->dk_norm_weight)
      return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: a norm weight and its gradient accumulator go together");
  } else if (a->q_norm_weight || a->k_norm_weight || a->dq_norm_weight || a->dk_norm_weight) {
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack_bwd: norm weights given without qk_norm");
  }
  RopeParams p = {};
  p.qkv = (const bf16*)a->dqkv;
  p.cos = a->cos;
  p.sin = a->sin;
  p.q = (bf16*)a->dq;
  p.k = (bf16*)a->dk;
  p.v = (bf16*)a->dv;
  p.Z = a->grid[0];
  p.Y = a->grid[1];
  p.X = a->grid[2];
  p.Zt = a->table_z;
  p.H = a->heads;
  p.D = a->head_dim;
  p.ld = a->dqkv_row_stride;
  p.M = (int64_t)a->batch * p.Z * p.Y * p.X;
  const int cph = a->layout == STRATA_HIP_ROPE_HALF ? p.D / 16 : p.D / 8;
  const int64_t total = p.M * p.H * cph;
  if (total == 0) return STRATA_HIP_OK;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "rope_qkv_pack_bwd: too many tokens");
  if (a->qk_norm) {
    p.x = (const bf16*)a->qkv;
    p.ldx = a->qkv_row_stride;
    p.eps = a->qk_norm_eps;
    p.qw = (const bf16*)a->q_norm_weight;
    p.kw = (const bf16*)a->k_norm_weight;
    p.dqw = a->dq_norm_weight;
    p.dkw = a->dk_norm_weight;
    // a bounded grid: the weight-gradient atomics are one per channel and block
    const unsigned nb = (unsigned)(blocks < 2048 ? blocks : 2048);
    if (a->layout == STRATA_HIP_ROPE_HALF)
      hipLaunchKernelGGL(rope_unpack_norm_kernel<true>, dim3(nb), dim3(256), 0, (hipStream_t)stream, p, total);
    else
      hipLaunchKernelGGL(rope_unpack_norm_kernel<false>, dim3(nb), dim3(256), 0, (hipStream_t)stream, p, total);
    return check_launch("rope_unpack_norm_kernel");
  }
  if (a->layout == STRATA_HIP_ROPE_HALF)
    hipLaunchKernelGGL(rope_unpack_half_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p, total);
  else
    hipLaunchKernelGGL(rope_unpack_inter_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p, total);
  return check_launch("rope_unpack_kernel");
}

extern "C" int strata_hip_rope_qkv_pack(const strata_hip_rope_pack_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: null args");
  if (!a->qkv || !a->cos || !a->sin || !a->k)
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: null pointer");  // q may be NULL: k (and v) only
  if (a->batch < 0 || a->grid[0] <= 0 || a->grid[1] <= 0 || a->grid[2] <= 0 || a->heads <= 0)
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: bad batch/grid/heads");
  if (a->table_z != 1 && a->table_z != a->grid[0])
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: table_z must be 1 or Z");
  if (a->layout != STRATA_HIP_ROPE_HALF && a->layout != STRATA_HIP_ROPE_INTERLEAVED)
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: bad layout");
  if (a->layout == STRATA_HIP_ROPE_HALF ? (a->head_dim % 16) : (a->head_dim % 8))
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: head_dim must be a multiple of 16 (half) or 8 (interleaved)");
  const int64_t C = (int64_t)a->heads * a->head_dim;
  if (a->qkv_row_stride < 3 * C || a->qkv_row_stride % 8)
    return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: qkv row stride must be >= 3*H*D and a multiple of 8");
  const void* ptrs[6] = {a->qkv, a->cos, a->sin, a->q, a->k, a->v};
  for (int i = 0; i < 6; ++i)
    if ((uintptr_t)ptrs[i] & 15) return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: pointers must be 16-byte aligned");
  RopeParams p;
  p.qkv = (const bf16*)a->qkv;
  p.cos = a->cos;
  p.sin = a->sin;
  p.q = (bf16*)a->q;
  p.k = (bf16*)a->k;
  p.v = (bf16*)a->v;
  p.Z = a->grid[0];
  p.Y = a->grid[1];
  p.X = a->grid[2];
  p.Zt = a->table_z;
  p.H = a->heads;
  p.D = a->head_dim;
  p.ld = a->qkv_row_stride;
  p.M = (int64_t)a->batch * p.Z * p.Y * p.X;
  const int cph = a->layout == STRATA_HIP_ROPE_HALF ? p.D / 16 : p.D / 8;
  if (a->qk_norm != 0 && a->qk_norm != 1) return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: qk_norm must be 0 or 1");
  if (a->qk_norm) {
    // the lanes of one head reduce by shuffles within an aligned power-of-two group
    if ((cph & (cph - 1)) || cph > 64)
      return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: qk_norm needs D/16 (half) or D/8 (interleaved) a power of two <= 64");
    if (!(a->qk_norm_eps >= 0.f)) return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: qk_norm_eps must be >= 0");
    if (((uintptr_t)a->q_norm_weight & 1) || ((uintptr_t)a->k_norm_weight & 1))
      return fail(STRATA_HIP_EINVAL, "rope_qkv_pack: norm weights must be 2-byte aligned");
  }
  p.qk_norm = a->qk_norm;
  p.eps = a->qk_norm_eps;
  p.qw = a->qk_norm ? (const bf16*)a->q_norm_weight : nullptr;
  p.kw = a->qk_norm ? (const bf16*)a->k_norm_weight : nullptr;
  const int64_t total = p.M * p.H * cph;
  if (total == 0) return STRATA_HIP_OK;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  if (blocks > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "rope_qkv_pack: too many tokens");
  if (a->layout == STRATA_HIP_ROPE_HALF) {
    const int64_t slice = ((total + ROPE_R - 1) / ROPE_R + 63) / 64 * 64;
    hipLaunchKernelGGL(rope_pack_half_kernel, dim3((unsigned)((slice + threads - 1) / threads)), dim3(threads), 0,
                       (hipStream_t)stream, p, total, slice);
  } else
    hipLaunchKernelGGL(rope_pack_inter_kernel, dim3((unsigned)blocks), dim3(threads), 0, (hipStream_t)stream, p, total);
  return check_launch("rope_pack_kernel");
}
