// NA3D backward for gfx950: dQ, dK, dV of natten.na3d (NATTEN 0.21.5's
// autograd function, which training reaches through train.py:1161), on the
// same clamped / dilated windows as the forward.
//
//   p_ij  = softmax_j(scale * q_i . k_j)      (j in the window W(i))
//   D_i   = sum_d dO_id * O_id
//   dS_ij = p_ij * (dO_i . v_j - D_i)
//   dQ_i  = scale * sum_{j in W(i)} dS_ij k_j
//   dK_j  = scale * sum_{i : j in W(i)} dS_ij q_i,   dV_j = sum_{i : j in W(i)} p_ij dO_i
//
// Three kernels, each a wave per 4 x 4 tile of tokens (4 lanes per token, D/4
// head dims per lane, dot products closed by two xor shuffles):
//   prep: per query, log2-sum-exp of its scores (recomputed: the forward keeps
//         no statistics) and D_i, into a caller-provided fp32 workspace;
//   dq:   per query, a walk over its window;
//   dkv:  per key, a walk over its inverse window {i : j in W(i)}, which per
//         axis is an interval (window starts are non-decreasing in i):
//         lo = 0 if j <= k - 1 else j - k + 1 + k/2,  hi = Lg - 1 if j >= Lg - k else j + k/2
//         (sub-grid coordinates of the dilation residue class).
// Scores run in log2 units (q pre-scaled by scale * log2 e), fp32 throughout;
// the neighbouring tokens of a tile share most of their window, so their
// K/V (or Q/dO) reads hit in L1/L2.  VALU-bound: no MFMA here.
#include "common.h"

namespace strata {

struct Na3dBwdParams {
  const void *q, *k, *v, *o, *dout;
  void *dq, *dk, *dv;
  float* lse;   // [B, Z, Y, X, H] log2-sum-exp of scale*log2(e)*q.k over the window
  float* dsum;  // [B, Z, Y, X, H] D_i
  int B, H, Z, Y, X;
  int ker[3], dil[3];
  float scale;
  int nyt, nxt;  // 4-row tiles along y, 16-column workgroup boxes along x
};

template <typename T, int DPL>
__device__ __forceinline__ void load_dims(const T* p, float (&f)[DPL]) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int i = 0; i < DPL; i += 8) {
      const u32x4 w = *(const u32x4*)(p + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[i + 2 * e] = bf16_lo(w[e]);
        f[i + 2 * e + 1] = bf16_hi(w[e]);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < DPL; i += 4) {
      const f32x4 w = *(const f32x4*)(p + i);
#pragma unroll
      for (int e = 0; e < 4; ++e) f[i + e] = w[e];
    }
  }
}

template <typename T, int DPL>
__device__ __forceinline__ void store_dims(T* p, const float (&f)[DPL], float mul) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int i = 0; i < DPL; i += 8) {
      const u32x4 w = {pack_bf16x2(f[i] * mul, f[i + 1] * mul), pack_bf16x2(f[i + 2] * mul, f[i + 3] * mul),
                       pack_bf16x2(f[i + 4] * mul, f[i + 5] * mul), pack_bf16x2(f[i + 6] * mul, f[i + 7] * mul)};
      *(u32x4*)(p + i) = w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < DPL; i += 4) *(f32x4*)(p + i) = (f32x4){f[i] * mul, f[i + 1] * mul, f[i + 2] * mul, f[i + 3] * mul};
  }
}

// Sum over the 4 lanes of a token.
__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 1);
  return x + __shfl_xor(x, 2);
}

template <int DPL>
__device__ __forceinline__ float dot(const float (&a)[DPL], const float (&b)[DPL]) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < DPL; ++i) s = fmaf(a[i], b[i], s);
  return s;
}

// The token of this lane: a workgroup is 4 waves side by side along x, each a
// 4 x 4 (y, x) tile of one (b, h, z); lane l holds dims [(l & 3) * D/4, +D/4)
// of token l >> 2 (row-major in the tile).
struct Tok {
  int b, h, z, y, x;
  bool valid;
};

__device__ __forceinline__ Tok token_of(const Na3dBwdParams& p) {
  int w = (int)blockIdx.x;
  const int xb = w % p.nxt;
  w /= p.nxt;
  const int yt = w % p.nyt;
  w /= p.nyt;
  const int z = w % p.Z;
  w /= p.Z;
  const int h = w % p.H;
  const int b = w / p.H;
  const int tid = (int)threadIdx.x;
  const int wave = tid >> 6, t = (tid & 63) >> 2;
  Tok k;
  k.b = b;
  k.h = h;
  k.z = z;
  k.y = yt * 4 + (t >> 2);
  k.x = xb * 16 + wave * 4 + (t & 3);
  k.valid = k.y < p.Y && k.x < p.X;
  if (!k.valid) {  // clamp so every address stays in range; nothing is stored
    k.y = min(k.y, p.Y - 1);
    k.x = min(k.x, p.X - 1);
  }
  return k;
}

__device__ __forceinline__ int64_t tok_index(const Na3dBwdParams& p, int b, int z, int y, int x, int h) {
  return ((((int64_t)b * p.Z + z) * p.Y + y) * p.X + x) * p.H + h;
}

// Window of coordinate c on one axis: first key and the key step.
__device__ __forceinline__ int axis_win_first(int c, int L, int k, int d) {
  const int g = c % d;
  return g + d * win_start(c / d, sub_len(L, g, d), k);
}

// Inverse window of key coordinate c on one axis: first query, query count (step d).
__device__ __forceinline__ void axis_inv(int c, int L, int k, int d, int& first, int& count) {
  const int g = c % d, j = c / d, Lg = sub_len(L, g, d), r = k / 2;
  const int lo = j - k + 1 <= 0 ? 0 : j - k + 1 + r;
  const int hi = j >= Lg - k ? Lg - 1 : j + r;
  first = g + d * lo;
  count = hi - lo + 1;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void na3d_bwd_prep_kernel(Na3dBwdParams p) {
  constexpr int DPL = D / 4;
  const Tok t = token_of(p);
  const int dq4 = (int)(threadIdx.x & 3) * DPL;
  const float c2 = p.scale * 1.4426950408889634f;
  const int64_t ti = tok_index(p, t.b, t.z, t.y, t.x, t.h);
  float qf[DPL], a[DPL], bv[DPL];
  load_dims<T, DPL>((const T*)p.q + ti * D + dq4, qf);
#pragma unroll
  for (int i = 0; i < DPL; ++i) qf[i] *= c2;
  load_dims<T, DPL>((const T*)p.dout + ti * D + dq4, a);
  load_dims<T, DPL>((const T*)p.o + ti * D + dq4, bv);
  const float dsum = quad_sum(dot(a, bv));

  const int z0 = axis_win_first(t.z, p.Z, p.ker[0], p.dil[0]);
  const int y0 = axis_win_first(t.y, p.Y, p.ker[1], p.dil[1]);
  const int x0 = axis_win_first(t.x, p.X, p.ker[2], p.dil[2]);
  float m = -INFINITY, l = 0.f;
  for (int a0 = 0; a0 < p.ker[0]; ++a0)
    for (int a1 = 0; a1 < p.ker[1]; ++a1)
      for (int a2 = 0; a2 < p.ker[2]; ++a2) {
        const int64_t kj = tok_index(p, t.b, z0 + a0 * p.dil[0], y0 + a1 * p.dil[1], x0 + a2 * p.dil[2], t.h);
        float kf[DPL];
        load_dims<T, DPL>((const T*)p.k + kj * D + dq4, kf);
        const float s = quad_sum(dot(qf, kf));
        const float mn = fmaxf(m, s);
        l = l * exp2f(m - mn) + exp2f(s - mn);
        m = mn;
      }
  if (t.valid && (threadIdx.x & 3) == 0) {
    p.lse[ti] = m + log2f(l);
    p.dsum[ti] = dsum;
  }
}

template <typename T, int D>
__global__ __launch_bounds__(256) void na3d_bwd_dq_kernel(Na3dBwdParams p) {
  constexpr int DPL = D / 4;
  const Tok t = token_of(p);
  const int dq4 = (int)(threadIdx.x & 3) * DPL;
  const float c2 = p.scale * 1.4426950408889634f;
  const int64_t ti = tok_index(p, t.b, t.z, t.y, t.x, t.h);
  float qf[DPL], dof[DPL], acc[DPL];
  load_dims<T, DPL>((const T*)p.q + ti * D + dq4, qf);
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    qf[i] *= c2;
    acc[i] = 0.f;
  }
  load_dims<T, DPL>((const T*)p.dout + ti * D + dq4, dof);
  const float lse = p.lse[ti], dsum = p.dsum[ti];

  const int z0 = axis_win_first(t.z, p.Z, p.ker[0], p.dil[0]);
  const int y0 = axis_win_first(t.y, p.Y, p.ker[1], p.dil[1]);
  const int x0 = axis_win_first(t.x, p.X, p.ker[2], p.dil[2]);
  for (int a0 = 0; a0 < p.ker[0]; ++a0)
    for (int a1 = 0; a1 < p.ker[1]; ++a1)
      for (int a2 = 0; a2 < p.ker[2]; ++a2) {
        const int64_t kj = tok_index(p, t.b, z0 + a0 * p.dil[0], y0 + a1 * p.dil[1], x0 + a2 * p.dil[2], t.h);
        float kf[DPL], vf[DPL];
        load_dims<T, DPL>((const T*)p.k + kj * D + dq4, kf);
        load_dims<T, DPL>((const T*)p.v + kj * D + dq4, vf);
        const float pr = exp2f(quad_sum(dot(qf, kf)) - lse);
        const float ds = pr * (quad_sum(dot(dof, vf)) - dsum);
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] = fmaf(ds, kf[i], acc[i]);
      }
  if (t.valid) store_dims<T, DPL>((T*)p.dq + ti * D + dq4, acc, p.scale);
}

template <typename T, int D>
__global__ __launch_bounds__(256) void na3d_bwd_dkv_kernel(Na3dBwdParams p) {
  constexpr int DPL = D / 4;
  const Tok t = token_of(p);
  const int dq4 = (int)(threadIdx.x & 3) * DPL;
  const float c2 = p.scale * 1.4426950408889634f;
  const int64_t tj = tok_index(p, t.b, t.z, t.y, t.x, t.h);
  float kf[DPL], vf[DPL], dk[DPL], dv[DPL];
  load_dims<T, DPL>((const T*)p.k + tj * D + dq4, kf);
  load_dims<T, DPL>((const T*)p.v + tj * D + dq4, vf);
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    kf[i] *= c2;
    dk[i] = 0.f;
    dv[i] = 0.f;
  }
  int zf, zn, yf, yn, xf, xn;
  axis_inv(t.z, p.Z, p.ker[0], p.dil[0], zf, zn);
  axis_inv(t.y, p.Y, p.ker[1], p.dil[1], yf, yn);
  axis_inv(t.x, p.X, p.ker[2], p.dil[2], xf, xn);
  for (int a0 = 0; a0 < zn; ++a0)
    for (int a1 = 0; a1 < yn; ++a1)
      for (int a2 = 0; a2 < xn; ++a2) {
        const int64_t qi = tok_index(p, t.b, zf + a0 * p.dil[0], yf + a1 * p.dil[1], xf + a2 * p.dil[2], t.h);
        float qf[DPL], dof[DPL];
        load_dims<T, DPL>((const T*)p.q + qi * D + dq4, qf);
        load_dims<T, DPL>((const T*)p.dout + qi * D + dq4, dof);
        const float pr = exp2f(quad_sum(dot(qf, kf)) - p.lse[qi]);
        const float ds = pr * (quad_sum(dot(dof, vf)) - p.dsum[qi]);
#pragma unroll
        for (int i = 0; i < DPL; ++i) {
          dv[i] = fmaf(pr, dof[i], dv[i]);
          dk[i] = fmaf(ds, qf[i], dk[i]);
        }
      }
  if (t.valid) {
    store_dims<T, DPL>((T*)p.dk + tj * D + dq4, dk, p.scale);
    store_dims<T, DPL>((T*)p.dv + tj * D + dq4, dv, 1.f);
  }
}

template <typename T, int D>
static int launch_bwd(const Na3dBwdParams& p, hipStream_t st) {
  const int64_t blocks = (int64_t)p.B * p.H * p.Z * p.nyt * p.nxt;
  if (blocks == 0) return STRATA_HIP_OK;
  if (blocks > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "na3d_bwd: problem too large for one launch");
  const dim3 grid((unsigned)blocks), block(256);
  hipLaunchKernelGGL((na3d_bwd_prep_kernel<T, D>), grid, block, 0, st, p);
  hipLaunchKernelGGL((na3d_bwd_dq_kernel<T, D>), grid, block, 0, st, p);
  hipLaunchKernelGGL((na3d_bwd_dkv_kernel<T, D>), grid, block, 0, st, p);
  return check_launch("na3d_bwd kernels");
}

template <typename T>
static int launch_bwd_t(const Na3dBwdParams& p, int D, hipStream_t st) {
  switch (D) {
    case 32: return launch_bwd<T, 32>(p, st);
    case 64: return launch_bwd<T, 64>(p, st);
    case 128: return launch_bwd<T, 128>(p, st);
    default: return fail(STRATA_HIP_EUNSUPPORTED, "na3d_bwd: head_dim must be 32, 64 or 128");
  }
}

static bool aligned16b(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace strata

using namespace strata;

extern "C" int strata_hip_na3d_bwd(const strata_hip_na3d_bwd_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "na3d_bwd: null args");
  if (a->dtype != STRATA_HIP_F32 && a->dtype != STRATA_HIP_BF16)
    return fail(STRATA_HIP_EINVAL, "na3d_bwd: dtype must be f32 or bf16");
  if (a->batch < 0 || a->heads <= 0 || a->head_dim <= 0)
    return fail(STRATA_HIP_EINVAL, "na3d_bwd: bad batch/heads/head_dim");
  static const char* axis = "zyx";
  for (int i = 0; i < 3; ++i) {
    const int L = a->grid[i], k = a->kernel[i], d = a->dilation[i];
    if (L <= 0) return fail(STRATA_HIP_EINVAL, std::string("na3d_bwd: grid size must be positive on axis ") + axis[i]);
    if (k <= 0 || (k % 2) == 0)
      return fail(STRATA_HIP_EINVAL, std::string("na3d_bwd: kernel size must be odd and positive on axis ") + axis[i]);
    if (d <= 0) return fail(STRATA_HIP_EINVAL, std::string("na3d_bwd: dilation must be positive on axis ") + axis[i]);
    if ((int64_t)d * k > L)
      return fail(STRATA_HIP_EINVAL, std::string("na3d_bwd: dilation * kernel exceeds the grid on axis ") + axis[i]);
  }
  if (a->batch == 0) return STRATA_HIP_OK;
  const void* ptrs[] = {a->q, a->k, a->v, a->out, a->dout, a->dq, a->dk, a->dv, a->workspace};
  for (const void* ptr : ptrs) {
    if (!ptr) return fail(STRATA_HIP_EINVAL, "na3d_bwd: null tensor pointer");
    if (!aligned16b(ptr)) return fail(STRATA_HIP_EINVAL, "na3d_bwd: tensors must be 16-byte aligned");
  }
  Na3dBwdParams p = {};
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.o = a->out;
  p.dout = a->dout;
  p.dq = a->dq;
  p.dk = a->dk;
  p.dv = a->dv;
  p.B = a->batch;
  p.H = a->heads;
  p.Z = a->grid[0];
  p.Y = a->grid[1];
  p.X = a->grid[2];
  for (int i = 0; i < 3; ++i) {
    p.ker[i] = a->kernel[i];
    p.dil[i] = a->dilation[i];
  }
  p.scale = a->scale;
  const int64_t tokens = (int64_t)p.B * p.Z * p.Y * p.X * p.H;
  p.lse = a->workspace;
  p.dsum = a->workspace + tokens;
  p.nyt = (p.Y + 3) / 4;
  p.nxt = (p.X + 15) / 16;
  hipStream_t st = (hipStream_t)stream;
  return a->dtype == STRATA_HIP_BF16 ? launch_bwd_t<bf16>(p, a->head_dim, st) : launch_bwd_t<float>(p, a->head_dim, st);
}
