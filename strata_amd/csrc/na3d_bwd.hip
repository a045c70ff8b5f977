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
// Three steps, prep, dq and dk/dv.  bf16 with head_dim 64, dilation 1 and
// kx <= 13 (the training shapes) runs MFMA versions that stage the
// workgroup's shared K/V or Q/dO rows in LDS; for ky in {5, 7}, kx <= 9,
// kz >= 3 (the block's windows) dq, dV and dK walk strips like the forward
// (the rows whose windows are not clamped) and the clamped edge rows walk
// tiles, all in one launch (na3d_bwd_small_fused_kernel).  The general VALU
// versions (4 lanes per token, D/4 head dims per lane, dot products closed by
// two xor shuffles) take everything else:
//   prep: per query, log2-sum-exp of its scores (recomputed, unless the caller
//         passes the forward's, strata_hip_na3d_fwd's lse output: then only
//         D_i) and D_i, into a caller-provided fp32 workspace;
//   dq:   per query, a walk over its window;
//   dkv:  per key, a walk over its inverse window {i : j in W(i)}, which per
//         axis is an interval (window starts are non-decreasing in i):
//         lo = 0 if j <= k - 1 else j - k + 1 + k/2,  hi = Lg - 1 if j >= Lg - k else j + k/2
//         (sub-grid coordinates of the dilation residue class).
// Scores run in log2 units (q, or in dk/dv k, pre-scaled by scale * log2 e),
// fp32 throughout.
#include <algorithm>
#include <cstdlib>
#include <mutex>

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
  int lse_given; // lse holds the forward's statistics: prep computes D_i only
  int qy0, qny;  // token rows [qy0, qy0 + qny) of the tile walks (0 and Y but for the dq edge rows)
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

// The token of in-tile index t (row r0 + (t >> 2), column t & 3) of this lane's
// wave, for workgroups of `rows` rows (nyt of them along y).
__device__ __forceinline__ Tok token_rows(const Na3dBwdParams& p, int wid, int nyt, int rows, int r0, int t) {
  int w = wid;
  const int xb = w % p.nxt;
  w /= p.nxt;
  const int yt = w % nyt;
  w /= nyt;
  const int z = w % p.Z;
  w /= p.Z;
  const int h = w % p.H;
  const int b = w / p.H;
  const int wave = (int)threadIdx.x >> 6;
  Tok k;
  k.b = b;
  k.h = h;
  k.z = z;
  k.y = p.qy0 + yt * rows + r0 + (t >> 2);
  k.x = xb * 16 + wave * 4 + (t & 3);
  k.valid = k.y < p.qy0 + p.qny && k.y < p.Y && k.x < p.X;
  if (!k.valid) {  // clamp so every address stays in range; nothing is stored
    k.y = min(k.y, p.Y - 1);
    k.x = min(k.x, p.X - 1);
  }
  return k;
}

// The token of in-tile index t (row t >> 2, column t & 3) of this lane's wave.
__device__ __forceinline__ Tok token_at(const Na3dBwdParams& p, int t) { return token_rows(p, (int)blockIdx.x, p.nyt, 4, 0, t); }

// VALU kernels: 4 lanes per token, lane l on token l >> 2.
__device__ __forceinline__ Tok token_of(const Na3dBwdParams& p) { return token_at(p, ((int)threadIdx.x & 63) >> 2); }

// LDS writes of this wave done (its own rows; no other wave reads them).
__device__ __forceinline__ void wait_lds() {
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (3 << 14));  // lgkmcnt(0), vmcnt/expcnt untouched
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
__host__ __device__ __forceinline__ void axis_inv(int c, int L, int k, int d, int& first, int& count) {
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

// ---------------------------------------------------------------------------
// MFMA prep for bf16, head_dim 64, dilation 1 (a backward without the
// forward's lse): a wave per 4 x 4 query tile walks its window union a key row
// at a time with the score MFMA only (S^T = K Q^T, keys on M straight from
// global memory).  Each lane keeps a running maximum and sum over the 4 keys
// of its query it sees per row; the four lanes of a query (g = 0..3) merge
// them at the end.  D_i = dO_i . O_i on the same lanes.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void na3d_bwd_prep_mfma_kernel(Na3dBwdParams p) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int D = 64, KS = 2;
  const int tid = (int)threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, n16 = lane & 15, g = lane >> 4;
  const Tok t = token_at(p, n16);
  const float c2 = p.scale * 1.4426950408889634f;
  const int kz = p.ker[0], ky = p.ker[1], kx = p.ker[2];
  const int64_t qi = tok_index(p, t.b, t.z, t.y, t.x, t.h);
  bf16x8 qreg[KS];
  float dsum = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qreg[ks] = *(const bf16x8*)((const bf16*)p.q + qi * D + 8 * (4 * ks + g));
    const bf16x8 a = *(const bf16x8*)((const bf16*)p.dout + qi * D + 8 * (4 * ks + g));
    const bf16x8 o = *(const bf16x8*)((const bf16*)p.o + qi * D + 8 * (4 * ks + g));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      qreg[ks][e] = (bf16)((float)qreg[ks][e] * c2);
      dsum = fmaf((float)a[e], (float)o[e], dsum);
    }
  }
  dsum += __shfl_xor(dsum, 16);
  dsum += __shfl_xor(dsum, 32);

  const int xw0 = min(((int)blockIdx.x % p.nxt) * 16 + wave * 4, p.X - 1);
  const int X0 = win_start(xw0, p.X, kx);
  const int sx = win_start(t.x, p.X, kx);
  f32x4 xb, ninf = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = X0 + 4 * g + i;
    xb[i] = (key >= sx && key < sx + kx) ? 0.f : -INFINITY;
  }
  const int kxl = min(X0 + n16, p.X - 1);
  const int ty0 = ((int)(blockIdx.x / p.nxt) % p.nyt) * 4;
  const int Yu0 = win_start(min(ty0, p.Y - 1), p.Y, ky);
  const int NR = win_start(min(ty0 + 3, p.Y - 1), p.Y, ky) + ky - Yu0;
  const int sy = win_start(t.y, p.Y, ky);
  const int sz = win_start(t.z, p.Z, kz);
  float m = -INFINITY, l = 0.f;
  for (int a0 = 0; a0 < kz; ++a0) {
    for (int r0 = 0; r0 < NR; ++r0) {
      const int yk = Yu0 + r0;
      const int64_t kj = tok_index(p, t.b, sz + a0, yk, kxl, t.h);
      f32x4 sc = (yk >= sy && yk < sy + ky) ? xb : ninf;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8*)((const bf16*)p.k + kj * D + 8 * (4 * ks + g)),
                                                     qreg[ks], sc, 0, 0, 0);
      const float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      const float mn = fmaxf(m, mx);
      if (mn > -INFINITY) {
        l = l * exp2f(m - mn) + exp2f(sc[0] - mn) + exp2f(sc[1] - mn) + exp2f(sc[2] - mn) + exp2f(sc[3] - mn);
        m = mn;
      }
    }
  }
  // merge the four lanes of the query
#pragma unroll
  for (int sh = 16; sh <= 32; sh *= 2) {
    const float mo = __shfl_xor(m, sh), lo = __shfl_xor(l, sh);
    const float mn = fmaxf(m, mo);
    l = (m > -INFINITY ? l * exp2f(m - mn) : 0.f) + (mo > -INFINITY ? lo * exp2f(mo - mn) : 0.f);
    m = mn;
  }
  if (t.valid && g == 0) {
    p.lse[qi] = m + log2f(l);
    p.dsum[qi] = dsum;
  }
#endif
}

// ---------------------------------------------------------------------------
// LDS-staged dk / dv for bf16, head_dim 64, dilation 1, kx <= 13.  The
// workgroup's 4 x 4 key tiles (four waves side by side along x, NT tiles per
// wave stacked along y: 16 key columns of one (b, h, z), 4 NT rows) share their
// queries: the union of the tiles' inverse windows is walked two
// query (z, y) rows at a time, each row's Q and dO over the workgroup's
// inverse-window columns (at most 16 + kx - 1 <= 28, staged as 32) copied into
// LDS once per workgroup by `buffer_load ... lds` (a ring of three stages),
// with the rows' log2-sum-exp and D_i beside them.  A wave takes its keys'
// 16-query block(s) of each staged row: S = Q K^T and dP = dO V^T with the
// tile's K (pre-scaled by scale * log2 e) and V as the register operand, the
// membership mask (key j in W(i) per axis, exact at clamped edges) as the C
// operand of S, P = 2^(S - lse), dS = P (dP - D); then dV^T += dO^T P and
// dK^T += Q^T dS over the row pair, with dO^T and Q^T read transposed
// (ds_read_b64_tr_b16).  A wave's keys near a grid edge can need up to 22
// queries along x: a second 16-query block then starts at most 16 columns
// before the stage's end and skips the columns the first one covered.  A tile
// none of whose keys lies in either staged row's windows skips the stage.
// ---------------------------------------------------------------------------
// 4x4 tiles per wave of the LDS kernels, stacked along y: two share each staged
// row pair between a wave's tiles (configs[1] 0.65 -> 0.62 ms, the configs[3]
// shape 2.31 -> 2.15 ms against one tile per wave).
constexpr int NA3D_BWD_NT = 2;

namespace dkvl {
constexpr int SW = 32;                     // staged query columns per row
constexpr int RB = SW * 64 * 2;            // bytes of one staged row of Q (or dO)
constexpr int NBUF = 3;                    // ring stages
constexpr int STAGE = 4 * RB + 4 * SW * 4;  // Q r0, Q r1, dO r0, dO r1, lse r0, r1, D r0, r1
}  // namespace dkvl

// `lds`: NBUF * STAGE bytes, 1 KiB aligned; `id`: the work unit (key tile box).
template <int NT>
__device__ __forceinline__ void na3d_bwd_dkv_lds_body(const Na3dBwdParams& p, int nyt, char* lds, int id) {
#if defined(__HIP_DEVICE_COMPILE__)
  using namespace dkvl;
  constexpr int D = 64, KS = 2, DB = 4;
  const int tid = (int)threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, n16 = lane & 15, g = lane >> 4;
  Tok t[NT];  // MFMA column n16 of tile tt = the lane's key in rows 4 tt .. 4 tt + 3 of the workgroup
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) t[tt] = token_rows(p, id, nyt, 4 * NT, 4 * tt, n16);
  const float c2 = p.scale * 1.4426950408889634f;
  const int kz = p.ker[0], ky = p.ker[1], kx = p.ker[2];
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

  int64_t kj[NT];
  bf16x8 kreg[NT][KS], vreg[NT][KS];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    kj[tt] = tok_index(p, t[tt].b, t[tt].z, t[tt].y, t[tt].x, t[tt].h);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kreg[tt][ks] = *(const bf16x8*)((const bf16*)p.k + kj[tt] * D + 8 * (4 * ks + g));
      vreg[tt][ks] = *(const bf16x8*)((const bf16*)p.v + kj[tt] * D + 8 * (4 * ks + g));
#pragma unroll
      for (int e = 0; e < 8; ++e) kreg[tt][ks][e] = (bf16)((float)kreg[tt][ks][e] * c2);
    }
  }
  const Tok& t0 = t[0];  // b, h, z and the key column are the same for every tile

  // ---- x: the workgroup's query columns [SX0, SX0 + SW) and this wave's blocks ----
  const int KX0 = (id % p.nxt) * 16;
  int f, n;
  axis_inv(min(KX0, p.X - 1), p.X, kx, 1, f, n);
  const int SX0 = f;
  const int kx0 = min(KX0 + wave * 4, p.X - 1), kx1 = min(kx0 + 3, p.X - 1);
  axis_inv(kx0, p.X, kx, 1, f, n);
  const int wlo = f;
  axis_inv(kx1, p.X, kx, 1, f, n);
  const int whi = f + n;                 // one past the wave's last query column
  const int bs0 = wlo - SX0;             // <= 12
  const int nxb = whi - wlo > 16 ? 2 : 1;
  const int bs1 = min(bs0 + 16, SW - 16);
  int bs[2] = {bs0, bs1};
  // x membership of the lane's key in the windows of the block's columns 4g..4g+3
  uint32_t xm[2];
#pragma unroll
  for (int xb = 0; xb < 2; ++xb) {
    xm[xb] = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int cl = bs[xb] + 4 * g + e;  // column within the stage
      const int qx = SX0 + cl;
      const int sx = win_start(min(qx, p.X - 1), p.X, kx);
      const bool in = qx < p.X && (xb == 0 || cl >= bs0 + 16) && t0.x >= sx && t0.x < sx + kx;
      xm[xb] |= in ? (1u << e) : 0u;
    }
  }
  // LDS offsets: Q / dO A-operand rows (column bs + n16) and transposed reads
  uint32_t aoff[2][KS], toff[2][DB];
#pragma unroll
  for (int xb = 0; xb < 2; ++xb) {
    const int col = bs[xb] + n16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) aoff[xb][ks] = (uint32_t)((col * D + 8 * ((4 * ks + g) ^ (col & 7))) * 2);
    const int colv = bs[xb] + 4 * g + (n16 >> 2), dq = n16 & 3;
#pragma unroll
    for (int db = 0; db < DB; ++db)
      toff[xb][db] = (uint32_t)((colv * D + 8 * ((2 * db + (dq >> 1)) ^ (colv & 7)) + 4 * (dq & 1)) * 2);
  }

  // ---- y, z: the query rows of the workgroup's keys ----
  const int ky0 = min(p.qy0 + (id / p.nxt % nyt) * 4 * NT, p.Y - 1), ky1 = min(ky0 + 4 * NT - 1, p.Y - 1);
  axis_inv(ky0, p.Y, ky, 1, f, n);
  const int QY0 = f;
  axis_inv(ky1, p.Y, ky, 1, f, n);
  const int NY = f + n - QY0;
  int QZ0, NZ;
  axis_inv(t0.z, p.Z, kz, 1, QZ0, NZ);
  const int nrows = NZ * NY;
  const int nst = (nrows + 1) / 2;

  // ---- copies: wave w stages query columns 8w .. 8w+7 of both rows of Q and dO;
  // waves 0 / 1 also the rows' lse / D (one dword per lane) ----
  const int64_t rowb = (int64_t)p.H * D * 2;  // bytes between neighbouring x tokens
  const uint32_t rec = (uint32_t)((int64_t)(p.X - 1) * rowb + D * 2);
  uint32_t voff;
  {
    const int cl = 8 * wave + (lane >> 3);
    const int qx = SX0 + cl;
    const int chunk = (lane & 7) ^ (cl & 7);
    voff = qx < p.X ? (uint32_t)(qx * rowb + 16 * chunk) : OOB;
  }
  const int scol = lane & 31;  // lse / D copies: lane -> (row lane >> 5, column lane & 31)
  const bool scol_in = SX0 + scol < p.X;
  const char* qbase = (const char*)p.q + 2 * (int64_t)t0.h * D;
  const char* obase = (const char*)p.dout + 2 * (int64_t)t0.h * D;
  const float* sbase = wave == 0 ? p.lse : p.dsum;
  auto row_tok = [&](int sr) {  // token index of (row sr, x = 0, head 0)
    const int zq = QZ0 + sr / NY, yq = QY0 + sr % NY;
    return (((int64_t)t0.b * p.Z + zq) * p.Y + yq) * p.X * p.H;
  };
  auto issue = [&](int s) {
    const uint32_t st = lds_base + (uint32_t)((s % NBUF) * STAGE);
    const int r0 = 2 * s, r1 = 2 * s + 1;
    const bool l0 = r0 < nrows, l1 = r1 < nrows;
    const int64_t w0 = l0 ? row_tok(r0) : 0, w1 = l1 ? row_tok(r1) : 0;
    dma_row16(make_rsrc(qbase + w0 * D * 2, l0 ? rec : 0u), st + 0 * RB + wave * 1024, voff);
    dma_row16(make_rsrc(qbase + w1 * D * 2, l1 ? rec : 0u), st + 1 * RB + wave * 1024, voff);
    dma_row16(make_rsrc(obase + w0 * D * 2, l0 ? rec : 0u), st + 2 * RB + wave * 1024, voff);
    dma_row16(make_rsrc(obase + w1 * D * 2, l1 ? rec : 0u), st + 3 * RB + wave * 1024, voff);
    if (wave < 2) {
      // row 1 sits (w1 - w0) tokens after row 0 in the [B, Z, Y, X, H] statistics
      const int64_t dt = l1 ? w1 - w0 : 0;
      const uint32_t so = (lane < 32 ? (l0 && scol_in) : (l1 && scol_in))
                              ? (uint32_t)(((lane < 32 ? 0 : dt) + (int64_t)(SX0 + scol) * p.H + t0.h) * 4)
                              : OOB;
      const uint32_t srec = l0 ? (uint32_t)((dt + (int64_t)p.X * p.H) * 4) : 0u;
      dma_dword(make_rsrc(sbase + w0, srec), st + 4 * RB + wave * 2 * SW * 4, so);
    }
  };

  f32x4 dk[NT][DB], dv[NT][DB];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int db = 0; db < DB; ++db) dk[tt][db] = dv[tt][db] = (f32x4){0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < NBUF - 1; ++s) issue(s);
  for (int s = 0; s < nst; ++s) {
    if (wave < 2)
      wait_vmcnt((NBUF - 2) * 5);
    else
      wait_vmcnt((NBUF - 2) * 4);
    lds_barrier();
    issue(s + NBUF - 1);
    const char* st = lds + (s % NBUF) * STAGE;
    const float* sl = (const float*)(st + 4 * RB);  // lse r0, lse r1, D r0, D r1
    // y / z membership of the lane's key (each tile) for the two rows; a tile none of
    // whose keys is in either row's windows skips the stage (wave-uniform)
    bool yz[NT][2], act[NT];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int sr = 2 * s + r;
      const int zq = QZ0 + sr / NY, yq = QY0 + sr % NY;
      const int wy = win_start(min(yq, p.Y - 1), p.Y, ky), wz = win_start(min(zq, p.Z - 1), p.Z, kz);
      const bool zin = sr < nrows && t0.z >= wz && t0.z < wz + kz;
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) yz[tt][r] = zin && t[tt].y >= wy && t[tt].y < wy + ky;
    }
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) act[tt] = __builtin_amdgcn_ballot_w64(yz[tt][0] || yz[tt][1]) != 0;
#pragma unroll
    for (int xb = 0; xb < 2; ++xb) {
      if (xb >= nxb) break;  // wave-uniform
      bf16x8 qa[2][KS], da[2][KS];
      float lse[2][4], dsm[2][4];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          qa[r][ks] = *(const bf16x8*)(st + r * RB + aoff[xb][ks]);
          da[r][ks] = *(const bf16x8*)(st + (2 + r) * RB + aoff[xb][ks]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int cl = bs[xb] + 4 * g + e;
          lse[r][e] = sl[r * SW + cl];
          dsm[r][e] = sl[(2 + r) * SW + cl];
        }
      }
      bf16x8 pbp[NT], pbs[NT];
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        if (!act[tt]) continue;
        float pv[2][4], sv[2][4];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          f32x4 sc, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int e = 0; e < 4; ++e) sc[e] = (yz[tt][r] && ((xm[xb] >> e) & 1)) ? 0.f : -INFINITY;
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[r][ks], kreg[tt][ks], sc, 0, 0, 0);
            dp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(da[r][ks], vreg[tt][ks], dp, 0, 0, 0);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pv[r][e] = __builtin_amdgcn_exp2f(sc[e] - lse[r][e]);
            sv[r][e] = pv[r][e] * (dp[e] - dsm[r][e]);
          }
        }
        pbp[tt] = __builtin_bit_cast(
            bf16x8, ((u32x4){pack_bf16x2(pv[0][0], pv[0][1]), pack_bf16x2(pv[0][2], pv[0][3]),
                             pack_bf16x2(pv[1][0], pv[1][1]), pack_bf16x2(pv[1][2], pv[1][3])}));
        pbs[tt] = __builtin_bit_cast(
            bf16x8, ((u32x4){pack_bf16x2(sv[0][0], sv[0][1]), pack_bf16x2(sv[0][2], sv[0][3]),
                             pack_bf16x2(sv[1][0], sv[1][1]), pack_bf16x2(sv[1][2], sv[1][3])}));
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const bf16x4 q0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, st + toff[xb][db]));
        const bf16x4 q1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, st + RB + toff[xb][db]));
        const bf16x4 o0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, st + 2 * RB + toff[xb][db]));
        const bf16x4 o1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, st + 3 * RB + toff[xb][db]));
        const bf16x8 qt = __builtin_shufflevector(q0, q1, 0, 1, 2, 3, 4, 5, 6, 7);
        const bf16x8 ot = __builtin_shufflevector(o0, o1, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) {
          if (!act[tt]) continue;
          dk[tt][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qt, pbs[tt], dk[tt][db], 0, 0, 0);
          dv[tt][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ot, pbp[tt], dv[tt][db], 0, 0, 0);
        }
      }
    }
  }
  wait_vmcnt(0);  // the ring's trailing (empty) stages
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    if (!t[tt].valid) continue;
    char* kp = (char*)p.dk + 2 * (kj[tt] * D) + 8 * g;
    char* vp = (char*)p.dv + 2 * (kj[tt] * D) + 8 * g;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      *(u32x2*)(kp + 32 * db) = (u32x2){pack_bf16x2(dk[tt][db][0] * p.scale, dk[tt][db][1] * p.scale),
                                        pack_bf16x2(dk[tt][db][2] * p.scale, dk[tt][db][3] * p.scale)};
      *(u32x2*)(vp + 32 * db) =
          (u32x2){pack_bf16x2(dv[tt][db][0], dv[tt][db][1]), pack_bf16x2(dv[tt][db][2], dv[tt][db][3])};
    }
  }
#endif
}

template <int NT>
__global__ __launch_bounds__(256, NT == 1 ? 3 : 2) void na3d_bwd_dkv_lds_kernel(Na3dBwdParams p, int nyt) {
  __shared__ __attribute__((aligned(1024))) char lds[dkvl::NBUF * dkvl::STAGE];
  na3d_bwd_dkv_lds_body<NT>(p, nyt, lds, (int)__builtin_amdgcn_workgroup_id_x());
}

// ---------------------------------------------------------------------------
// LDS-staged dq for bf16, head_dim 64, dilation 1, kx <= 13: the forward's
// walk for the workgroup's 4 x 4 query tiles (four waves along x, NT per wave
// along y: 16 query columns of one (b, h, z), 4 NT rows).  The union of their
// windows is walked two key (z, y)
// rows at a time, each row's K and V over the workgroup's window columns (at
// most 16 + kx - 1 <= 28, staged as 32) copied into LDS once per workgroup
// (`buffer_load ... lds`, a ring of three stages).  A wave takes its tile's
// 16-key block of each row (4 + kx - 1 <= 16 keys): S^T = K Q^T and dP^T =
// V dO^T with Q (pre-scaled by scale * log2 e) and dO as the register operand,
// the membership mask as the C operand of S^T, P^T = 2^(S^T - lse),
// dS^T = P^T (dP^T - D); then dQ^T += K^T dS^T over the row pair with K^T
// read transposed (ds_read_b64_tr_b16).  A tile whose queries see neither
// staged row skips the stage.
// ---------------------------------------------------------------------------
namespace dql {
constexpr int SW = 32;          // staged key columns per row
constexpr int RB = SW * 64 * 2;  // bytes of one staged row of K (or V)
constexpr int NBUF = 3;
constexpr int STAGE = 4 * RB;    // K r0, K r1, V r0, V r1
}  // namespace dql

// `lds`: NBUF * STAGE bytes, 1 KiB aligned; `id`: the work unit (query tile box).
template <int NT>
__device__ __forceinline__ void na3d_bwd_dq_lds_body(const Na3dBwdParams& p, int nyt, char* lds, int id) {
#if defined(__HIP_DEVICE_COMPILE__)
  using namespace dql;
  constexpr int D = 64, KS = 2, DB = 4;
  const int tid = (int)threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, n16 = lane & 15, g = lane >> 4;
  Tok t[NT];  // MFMA column n16 of tile tt = the lane's query in rows 4 tt .. 4 tt + 3 of the workgroup
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) t[tt] = token_rows(p, id, nyt, 4 * NT, 4 * tt, n16);
  const float c2 = p.scale * 1.4426950408889634f;
  const int kz = p.ker[0], ky = p.ker[1], kx = p.ker[2];
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

  int64_t qi[NT];
  bf16x8 qreg[NT][KS], doreg[NT][KS];
  float lse[NT], dsum[NT];
  int sy[NT];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    qi[tt] = tok_index(p, t[tt].b, t[tt].z, t[tt].y, t[tt].x, t[tt].h);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qreg[tt][ks] = *(const bf16x8*)((const bf16*)p.q + qi[tt] * D + 8 * (4 * ks + g));
      doreg[tt][ks] = *(const bf16x8*)((const bf16*)p.dout + qi[tt] * D + 8 * (4 * ks + g));
#pragma unroll
      for (int e = 0; e < 8; ++e) qreg[tt][ks][e] = (bf16)((float)qreg[tt][ks][e] * c2);
    }
    lse[tt] = p.lse[qi[tt]];
    dsum[tt] = p.dsum[qi[tt]];
    sy[tt] = win_start(t[tt].y, p.Y, ky);
  }
  const Tok& t0 = t[0];  // b, h, z and the query column are the same for every tile

  // ---- x: the workgroup's key columns [SX0, SX0 + SW) and this wave's block ----
  const int QX0 = (id % p.nxt) * 16;
  const int SX0 = win_start(min(QX0, p.X - 1), p.X, kx);
  const int qx0 = min(QX0 + wave * 4, p.X - 1);
  const int bs = win_start(qx0, p.X, kx) - SX0;  // <= 12
  const int sx = win_start(t0.x, p.X, kx);
  uint32_t xm = 0;  // bit e: key column bs + 4g + e is in the lane's query window
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int kc = SX0 + bs + 4 * g + e;
    xm |= (kc >= sx && kc < sx + kx) ? (1u << e) : 0u;
  }
  uint32_t aoff[KS], toff[DB];
  {
    const int col = bs + n16;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) aoff[ks] = (uint32_t)((col * D + 8 * ((4 * ks + g) ^ (col & 7))) * 2);
    const int colv = bs + 4 * g + (n16 >> 2), dq = n16 & 3;
#pragma unroll
    for (int db = 0; db < DB; ++db)
      toff[db] = (uint32_t)((colv * D + 8 * ((2 * db + (dq >> 1)) ^ (colv & 7)) + 4 * (dq & 1)) * 2);
  }

  // ---- y, z: the key rows of the workgroup's queries ----
  const int ty0 = p.qy0 + (id / p.nxt % nyt) * 4 * NT;
  const int KY0 = win_start(min(ty0, p.Y - 1), p.Y, ky);
  const int NY = win_start(min(ty0 + 4 * NT - 1, p.Y - 1), p.Y, ky) + ky - KY0;
  const int KZ0 = win_start(t0.z, p.Z, kz);
  const int nrows = kz * NY;
  const int nst = (nrows + 1) / 2;

  // ---- copies: wave w stages key columns 8w .. 8w+7 of both rows of K and V ----
  const int64_t rowb = (int64_t)p.H * D * 2;
  const uint32_t rec = (uint32_t)((int64_t)(p.X - 1) * rowb + D * 2);
  uint32_t voff;
  {
    const int cl = 8 * wave + (lane >> 3);
    const int kc = SX0 + cl;
    const int chunk = (lane & 7) ^ (cl & 7);
    voff = kc < p.X ? (uint32_t)(kc * rowb + 16 * chunk) : OOB;
  }
  const char* kbase = (const char*)p.k + 2 * (int64_t)t0.h * D;
  const char* vbase = (const char*)p.v + 2 * (int64_t)t0.h * D;
  auto row_tok = [&](int sr) {
    const int zk = KZ0 + sr / NY, yk = KY0 + sr % NY;
    return (((int64_t)t0.b * p.Z + zk) * p.Y + yk) * p.X * p.H;
  };
  auto issue = [&](int s) {
    const uint32_t st = lds_base + (uint32_t)((s % NBUF) * STAGE);
    const int r0 = 2 * s, r1 = 2 * s + 1;
    const bool l0 = r0 < nrows, l1 = r1 < nrows;
    const int64_t w0 = l0 ? row_tok(r0) : 0, w1 = l1 ? row_tok(r1) : 0;
    dma_row16(make_rsrc(kbase + w0 * D * 2, l0 ? rec : 0u), st + 0 * RB + wave * 1024, voff);
    dma_row16(make_rsrc(kbase + w1 * D * 2, l1 ? rec : 0u), st + 1 * RB + wave * 1024, voff);
    dma_row16(make_rsrc(vbase + w0 * D * 2, l0 ? rec : 0u), st + 2 * RB + wave * 1024, voff);
    dma_row16(make_rsrc(vbase + w1 * D * 2, l1 ? rec : 0u), st + 3 * RB + wave * 1024, voff);
  };

  f32x4 acc[NT][DB];
#pragma unroll
  for (int tt = 0; tt < NT; ++tt)
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[tt][db] = (f32x4){0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int s = 0; s < NBUF - 1; ++s) issue(s);
  for (int s = 0; s < nst; ++s) {
    wait_vmcnt((NBUF - 2) * 4);
    lds_barrier();
    issue(s + NBUF - 1);
    const char* st = lds + (s % NBUF) * STAGE;
    // y membership of the two key rows in each tile's query windows (z: every staged
    // plane is in the window); a tile with neither row in any window skips the stage
    bool yin[NT][2], act[NT];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int sr = 2 * s + r;
      const int yk = KY0 + sr % NY;
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) yin[tt][r] = sr < nrows && yk >= sy[tt] && yk < sy[tt] + ky;
    }
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) act[tt] = __builtin_amdgcn_ballot_w64(yin[tt][0] || yin[tt][1]) != 0;
    bf16x8 ka[2][KS], va[2][KS];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        ka[r][ks] = *(const bf16x8*)(st + r * RB + aoff[ks]);
        va[r][ks] = *(const bf16x8*)(st + (2 + r) * RB + aoff[ks]);
      }
    bf16x8 pb[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      if (!act[tt]) continue;
      float ds[2][4];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        f32x4 sc, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[e] = (yin[tt][r] && ((xm >> e) & 1)) ? 0.f : -INFINITY;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[r][ks], qreg[tt][ks], sc, 0, 0, 0);
          dp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[r][ks], doreg[tt][ks], dp, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) ds[r][e] = __builtin_amdgcn_exp2f(sc[e] - lse[tt]) * (dp[e] - dsum[tt]);
      }
      pb[tt] = __builtin_bit_cast(
          bf16x8, ((u32x4){pack_bf16x2(ds[0][0], ds[0][1]), pack_bf16x2(ds[0][2], ds[0][3]),
                           pack_bf16x2(ds[1][0], ds[1][1]), pack_bf16x2(ds[1][2], ds[1][3])}));
    }
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, st + toff[db]));
      const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, st + RB + toff[db]));
      const bf16x8 kt = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
        if (act[tt]) acc[tt][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt, pb[tt], acc[tt][db], 0, 0, 0);
    }
  }
  wait_vmcnt(0);  // the ring's trailing (empty) stages
#pragma unroll
  for (int tt = 0; tt < NT; ++tt) {
    if (!t[tt].valid) continue;
    char* op = (char*)p.dq + 2 * (qi[tt] * D) + 8 * g;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const u32x2 w = {pack_bf16x2(acc[tt][db][0] * p.scale, acc[tt][db][1] * p.scale),
                       pack_bf16x2(acc[tt][db][2] * p.scale, acc[tt][db][3] * p.scale)};
      *(u32x2*)(op + 32 * db) = w;
    }
  }
#endif
}

template <int NT>
__global__ __launch_bounds__(256, NT == 1 ? 3 : 2) void na3d_bwd_dq_lds_kernel(Na3dBwdParams p, int nyt) {
  __shared__ __attribute__((aligned(1024))) char lds[dql::NBUF * dql::STAGE];
  na3d_bwd_dq_lds_body<NT>(p, nyt, lds, (int)__builtin_amdgcn_workgroup_id_x());
}

// ---------------------------------------------------------------------------
// dq on regular strips (bf16, head_dim 64, dilation 1, kx <= 9, ky in {5, 7},
// kz >= 2): the forward's small-window strip walk.  A workgroup of four waves
// side by side in x (8 query columns each) walks one (b, h, z) column of 2 x 8
// query tiles down the query rows whose y window is not clamped; the key rows
// of the windows stream once per workgroup through a two-stage LDS ring (two
// 40-key rows of K, then of V, per stage; the kz slices of a row group back to
// back), and each wave keeps NS = (ky + 1) / 2 tiles in flight, tile j in slot
// j % NS: tile j's y-union is row groups j .. j + NS - 1, so in group gr the
// tile in its first group is in slot gr % NS and the one in its last group in
// slot (gr + 1) % NS, and the y masks are compile-time (query row t sees row r
// of its first group for r >= t and of its last for r <= t).  Per slot and
// stage: S^T = K Q^T (Q pre-scaled by scale * log2 e, the x window as the C
// operand) and dP^T = V dO^T, P^T = 2^(S^T - lse), dS^T = P^T (dP^T - D), then
// dQ^T += K^T dS^T with K^T read transposed.  P <= 1 (lse is the query's true
// log-sum-exp), so no range check is needed.  Q, dO, lse and D of the next
// tile are copied into LDS by `buffer_load ... lds` during the second slice of
// a group.  The clamped rows at the y edges go to na3d_bwd_dq_lds_kernel.
// ---------------------------------------------------------------------------
struct BwdStrips {
  int nxt;     // 32-column boxes along x
  int nch;     // y chunks per (b, h, z) column
  int cty;     // 2-row tiles per chunk
  int y0, y1;  // the strip rows [y0, y1): windows not clamped in y
  int total;   // workgroups
};

namespace dqs {
constexpr int NWX = 4, TX = 8, TY = 2, RPS = 2, NBUF = 2, D = 64, KS = 2, DB = 4, CPK = 8, KPK = 8;
constexpr int LW = (NWX - 1) * TX + 16;    // 40 keys of a staged row
constexpr int RB = LW * D * 2;             // bytes of one (tensor, row) region
constexpr int STAGE_B = 2 * RPS * RB;      // K rows 0..1, then V rows 0..1
constexpr int LPT = STAGE_B / 1024 / NWX;  // 1-KiB copies per wave per stage
constexpr int QWB = 16 * D * 2;            // one wave's 16 rows of Q (or dO)
constexpr int TWB = 2 * QWB + 2 * 256;     // per wave: Q, dO, then lse and D (one dword row each)
constexpr int QTB = NWX * TWB;
constexpr int RING_B = NBUF * STAGE_B;
constexpr int LDS_B = RING_B + QTB;
static_assert(LPT * NWX * 1024 == STAGE_B && 2 * LPT * 1024 == RPS * RB, "waves 0-1 copy K, 2-3 copy V");
static_assert(LW % 8 == 0, "rows start at whole swizzle periods");
static_assert(QTB <= RING_B, "tile 0's operands are staged through the ring");
}  // namespace dqs

// `lds`: dqs::LDS_B bytes, 1 KiB aligned; `id`: the work unit in [0, sg.total).
template <int KY>
__device__ __forceinline__ void na3d_bwd_dq_strip_body(const Na3dBwdParams& p, const BwdStrips& sg, char* lds, int id) {
#if defined(__HIP_DEVICE_COMPILE__)
  using namespace dqs;
  constexpr int NS = (TY + KY - 1) / RPS;  // tile slots per wave
  constexpr int KR = KY / 2;
  static_assert(TY + KY - 1 == NS * RPS, "one tile starts per row group");

  // ---- work unit: x box fastest, then z, chunk, head, batch ----
  int t = xcd_tile_order(sg.total, id);
  const int xb = t % sg.nxt;
  t /= sg.nxt;
  const int z = t % p.Z;
  t /= p.Z;
  const int ch = t % sg.nch;
  t /= sg.nch;
  const int h = t % p.H;
  const int b = t / p.H;
  const int ys = sg.y0 + ch * sg.cty * TY;
  const int ye = min(ys + sg.cty * TY, sg.y1);
  const int x0 = xb * (NWX * TX);
  if (ys >= ye) return;  // uniform over the workgroup
  const int NT = (ye - ys + TY - 1) / TY;
  const int S = ys - KR;            // first key row of tile 0's union
  const int NR = ye - ys + 2 * KR;  // key rows the strip streams
  const int NG = (NR + RPS - 1) / RPS;
  const int kz = p.ker[0], kx = p.ker[2];
  const int sz = win_start(z, p.Z, kz);
  const int X0 = win_start(min(x0, p.X - 1), p.X, kx);

  const int tid = (int)__builtin_amdgcn_workitem_id_x();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n16 = lane & 15;
  const int g = lane >> 4;
  const int trow = n16 / TX;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

  // ---- x geometry of the wave and of this lane's query ----
  const int xw0 = x0 + wave * TX;
  const int off_w = win_start(min(xw0, p.X - 1), p.X, kx) - X0;  // the wave's 16-key block in the staged row
  const int qx = xw0 + n16 % TX;
  f32x4 xbias;  // 0 or -inf: key 4g + i of the block inside / outside this lane's x window
  {
    const int sx = win_start(min(qx, p.X - 1), p.X, kx);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kc = X0 + off_w + 4 * g + i;
      xbias[i] = kc >= sx && kc < sx + kx ? 0.f : -INFINITY;
    }
  }
  const float c2 = p.scale * 1.4426950408889634f;

  // ---- tensor geometry (contiguous [B, Z, Y, X, H, D]) ----
  const int64_t colb = (int64_t)p.H * D * 2;  // bytes per x step
  const int64_t rowb = (int64_t)p.X * colb;   // per y row
  const int64_t zb = (int64_t)p.Y * rowb;     // per z slice
  const int64_t slice = ((int64_t)b * p.Z + z) * zb + (int64_t)h * D * 2;  // (b, z, h) of the queries

  // ---- K/V ring: stage-flat key f = row * LW + x, chunk slots swizzled by f & 7 ----
  const bool vwave = wave >= 2;
  uint32_t doff[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int f = ((wave & 1) * LPT + i) * KPK + lane / CPK;
    const int row = f / LW, key = f % LW;
    const int c = (lane % CPK) ^ (f & 7);
    doff[i] = X0 + key < p.X ? (uint32_t)(row * rowb + (int64_t)(X0 + key) * colb + 16 * c) : OOB;
  }
  const char* kvseg = (const char*)(vwave ? p.v : p.k) + ((int64_t)b * p.Z + sz) * zb + (int64_t)h * D * 2 +
                      (int64_t)S * rowb;
  int cz = 0, cp = 0;
  uint32_t issue_off = 0;
  auto issue = [&]() {
    const int nrow = min(max(NR - RPS * cp, 0), RPS);
    const u32x4 rs = make_rsrc(kvseg + (int64_t)cp * RPS * rowb + (int64_t)cz * zb, (uint32_t)(nrow * rowb));
    const uint32_t m0 = lds_base + issue_off + (uint32_t)wave * (LPT * 1024);
#pragma unroll
    for (int i = 0; i < LPT; ++i) dma_row16(rs, m0 + i * 1024, doff[i]);
    issue_off = issue_off + STAGE_B == RING_B ? 0 : issue_off + STAGE_B;
    if (++cz == kz) {
      cz = 0;
      ++cp;
    }
  };

  // ---- Q, dO, lse and D of a tile: one (b, z, h) slice, 31-bit offsets ----
  // (the record counts end at the slice, so the OOB offsets of idle lanes read zeros)
  const uint32_t qrec = (uint32_t)(zb - (int64_t)h * D * 2);
  const u32x4 rq = make_rsrc((const char*)p.q + slice, qrec);
  const u32x4 rd = make_rsrc((const char*)p.dout + slice, qrec);
  const int64_t sslice = ((int64_t)b * p.Z + z) * p.Y * p.X * p.H + h;  // (b, z, h) of the statistics
  const uint32_t srec = (uint32_t)(((int64_t)p.Y * p.X * p.H - h) * 4);
  const u32x4 rl = make_rsrc(p.lse + sslice, srec);
  const u32x4 rs2 = make_rsrc(p.dsum + sslice, srec);
  auto dma_tile = [&](int j, uint32_t off) {
    const int yt0 = ys + TY * j;
    const uint32_t m0 = lds_base + off + (uint32_t)wave * TWB;
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      const int n = lane / CPK + i * (64 / CPK);
      const int qy = min(yt0 + n / TX, ye - 1), cx = min(xw0 + n % TX, p.X - 1);
      const uint32_t o = (uint32_t)(qy * rowb + cx * colb) + 16 * (lane % CPK);
      dma_row16(rq, m0 + i * 1024, o);
      dma_row16(rd, m0 + QWB + i * 1024, o);
    }
    const int qy = min(yt0 + n16 / TX, ye - 1), cx = min(xw0 + n16 % TX, p.X - 1);
    const uint32_t so = lane < 16 ? (uint32_t)(((int64_t)qy * p.X + cx) * p.H * 4) : OOB;
    dma_dword(rl, m0 + 2 * QWB, so);
    dma_dword(rs2, m0 + 2 * QWB + 256, so);
  };

  // ---- LDS read offsets within row 0 of a stage (row r adds r * RB) ----
  uint32_t koff[KS], toff[DB];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int key = off_w + n16;
    koff[ks] = (key * D + 8 * ((4 * ks + g) ^ (key & 7))) * 2;
  }
  {
    const int keyv = off_w + 4 * g + (n16 >> 2), dq = n16 & 3;
#pragma unroll
    for (int db = 0; db < DB; ++db)
      toff[db] = (keyv * D + 8 * ((2 * db + (dq >> 1)) ^ (keyv & 7)) + 4 * (dq & 1)) * 2;
  }

  // ---- tile slots ----
  bf16x8 qreg[NS][KS], doreg[NS][KS];
  float lsev[NS], dsv[NS];
  f32x4 acc[NS][DB];
  const bool ylo = trow > 0;  // first group: row 0 masked for query row 1
  const bool yhi = trow < 1;  // last group: row 1 masked for query row 0

  auto start_tile = [&](int k, uint32_t off) {
    const char* qb = lds + off + wave * TWB;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qreg[k][ks] = *(const bf16x8*)(qb + n16 * D * 2 + (4 * ks + g) * 16);
      doreg[k][ks] = *(const bf16x8*)(qb + QWB + n16 * D * 2 + (4 * ks + g) * 16);
#pragma unroll
      for (int e = 0; e < 8; ++e) qreg[k][ks][e] = (bf16)((float)qreg[k][ks][e] * c2);
    }
    lsev[k] = *(const float*)(qb + 2 * QWB + 4 * n16);
    dsv[k] = *(const float*)(qb + 2 * QWB + 256 + 4 * n16);
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[k][db] = (f32x4){0.f, 0.f, 0.f, 0.f};
  };
  char* dqb = (char*)p.dq + slice + 8 * g;
  auto finish_tile = [&](int k, int j) {
    const int qy = ys + TY * j + trow;
    if (qy < ye && qx < p.X) {
      char* op = dqb + (int64_t)qy * rowb + (int64_t)qx * colb;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const u32x2 w = {pack_bf16x2(acc[k][db][0] * p.scale, acc[k][db][1] * p.scale),
                         pack_bf16x2(acc[k][db][2] * p.scale, acc[k][db][3] * p.scale)};
        *(u32x2*)(op + 32 * db) = w;
      }
    }
  };

  // One stage's math for every live slot.  C: slot of the tile in its first
  // group; ACT: bit k set if slot k holds a tile.
  auto stage_math = [&](auto cst, auto act, const bf16x8 (&ak)[RPS][KS], const bf16x8 (&vk)[RPS][KS],
                        const bf16x8 (&kt)[DB]) {
    constexpr int C = decltype(cst)::value;
    constexpr int ACT = decltype(act)::value;
    static_for<NS>([&](auto ttc) {
      constexpr int tt = decltype(ttc)::value;  // 0: the tile's first group, 1: its last
      constexpr int k = (C + tt) % NS;
      if constexpr ((ACT >> k) & 1) {
        float ds[RPS][4];
#pragma unroll
        for (int r = 0; r < RPS; ++r) {
          f32x4 sc = xbias, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[r][ks], qreg[k][ks], sc, 0, 0, 0);
            dp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vk[r][ks], doreg[k][ks], dp, 0, 0, 0);
          }
          const bool masked = (tt == 0 && r == 0 && ylo) || (tt == 1 && r == 1 && yhi);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            ds[r][e] = masked ? 0.f : __builtin_amdgcn_exp2f(sc[e] - lsev[k]) * (dp[e] - dsv[k]);
        }
        const bf16x8 pb = __builtin_bit_cast(
            bf16x8, ((u32x4){pack_bf16x2(ds[0][0], ds[0][1]), pack_bf16x2(ds[0][2], ds[0][3]),
                             pack_bf16x2(ds[1][0], ds[1][1]), pack_bf16x2(ds[1][2], ds[1][3])}));
#pragma unroll
        for (int db = 0; db < DB; ++db)
          acc[k][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[db], pb, acc[k][db], 0, 0, 0);
      }
    });
  };

  // Tile 0's operands are staged through the ring before the ring starts.
  dma_tile(0, 0);
  wait_vmcnt(0);
  start_tile(0, 0);
  wait_lgkm0();
  lds_barrier();  // tile 0's operands read before the ring overwrites them
#pragma unroll
  for (int s = 0; s < NBUF - 1; ++s) issue();

  uint32_t cur_off = 0;
  // Group gr: slot gr % NS starts tile gr, slot (gr + 1) % NS finishes tile gr - NS + 1.
  auto group = [&](auto cst, auto act, int gr) {
    constexpr int C = decltype(cst)::value;
    for (int zc = 0; zc < kz; ++zc) {
      const bool starting = zc == 0 && gr > 0 && gr < NT;
      if (starting)
        wait_vmcnt(0);  // the tile's operand copies as well
      else
        wait_vmcnt((NBUF - 2) * LPT);
      lds_barrier();
      issue();
      if (starting) start_tile(C, (uint32_t)RING_B);
      if (zc == 1 && gr + 1 < NT) dma_tile(gr + 1, (uint32_t)RING_B);
      const char* st = lds + cur_off;
      bf16x8 ak[RPS][KS], vk[RPS][KS], kt[DB];
#pragma unroll
      for (int r = 0; r < RPS; ++r)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          ak[r][ks] = *(const bf16x8*)(st + r * RB + koff[ks]);
          vk[r][ks] = *(const bf16x8*)(st + (RPS + r) * RB + koff[ks]);
        }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, st + toff[db]));
        const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, st + RB + toff[db]));
        kt[db] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
      stage_math(cst, act, ak, vk, kt);
      cur_off = cur_off + STAGE_B == RING_B ? 0 : cur_off + STAGE_B;
    }
    const int jf = gr - (NS - 1);
    if (jf >= 0 && jf < NT) finish_tile((C + 1) % NS, jf);
  };
  using ALL = std::integral_constant<int, (1 << NS) - 1>;
  static_for<NS - 1>([&](auto ig) {  // ramp-up: only the slots already holding a tile
    constexpr int G = decltype(ig)::value;
    group(std::integral_constant<int, G>{}, std::integral_constant<int, (1 << (G + 1)) - 1>{}, G);
  });
  for (int gr = NS - 1;; gr += NS) {  // NG = NT + NS - 1 >= NS
    bool done = false;
    static_for<NS>([&](auto ii) {
      constexpr int I = decltype(ii)::value;
      if (!done) {
        group(std::integral_constant<int, (NS - 1 + I) % NS>{}, ALL{}, gr + I);
        done = gr + I + 1 >= NG;
      }
    });
    if (done) break;
  }
  wait_vmcnt(0);  // the ring's trailing (empty) stages
#endif
}

// ---------------------------------------------------------------------------
// dK or dV on regular strips (bf16, head_dim 64, dilation 1, kx <= 9,
// ky in {5, 7}, kz >= 3): the strip walk with the roles of queries and keys
// swapped.  A workgroup of four waves side by side in x (8 key columns each)
// walks one (b, h, z) column of 2 x 8 key tiles down the key rows that no
// clamped query window reaches (rows [2 r + 1, Y - 2 r - 1), r = ky / 2), so
// that query row y sees key row y' exactly when |y - y'| <= r; the query rows
// of their inverse windows stream once per workgroup through a two-stage LDS
// ring (two 40-column rows of Q, then of dO, then the rows' lse and D), over
// the query slices whose z windows hold the key slice.  Each wave keeps
// NS = (ky + 1) / 2 tiles in flight with compile-time y masks, exactly as the
// forward strip (key row t sees query row r of its first group for r >= t and
// of its last for r <= t).  Per slot and stage, with the key tile as the
// register operand (K pre-scaled by scale * log2 e): S = Q K^T, P = 2^(S - lse)
// (x membership as the C operand), then
//   DK = 0:  dV^T += dO^T P;
//   DK = 1:  dP = dO V^T, dS = P (dP - D), dK^T += Q^T dS  (dK = scale * dK^T^T),
// with dO^T and Q^T read transposed.  dK and dV are separate launches: one
// kernel holding K, V and both accumulators for every slot would need more
// registers than a wave has at two waves per SIMD.  A wave's query block is
// the 16 columns from the first query whose window holds the wave's first key
// column; the host checks that it covers the inverse windows of all 8 columns.
// ---------------------------------------------------------------------------
namespace dkvs {
constexpr int NWX = 4, TX = 8, TY = 2, RPS = 2, NBUF = 2, D = 64, KS = 2, DB = 4, CPK = 8, KPK = 8;
constexpr int LW = 40;                     // staged query columns per row
constexpr int RB = LW * D * 2;             // bytes of one (tensor, row) region
constexpr int SB = 256;                    // one row of lse (or D): 64 dwords, 40 used
constexpr int STAGE_B = 2 * RPS * RB + 2 * RPS * SB;  // Q r0, r1, dO r0, r1, lse r0, r1, D r0, r1
constexpr int LPT = 2 * RPS * RB / 1024 / NWX;         // 1-KiB copies per wave per stage
constexpr int KWB = 16 * D * 2;            // one wave's 16 keys of K (or V)
constexpr int TWB = 2 * KWB;               // per wave: K, V of the next tile
constexpr int QTB = NWX * TWB;
constexpr int RING_B = NBUF * STAGE_B;
constexpr int LDS_B = RING_B + QTB;
static_assert(LPT * NWX * 1024 == 2 * RPS * RB && 2 * LPT * 1024 == RPS * RB, "waves 0-1 copy Q, 2-3 copy dO");
static_assert(QTB <= RING_B && STAGE_B % 1024 == 0, "stage layout");
}  // namespace dkvs

// `lds`: dkvs::LDS_B bytes, 1 KiB aligned; `id`: the work unit in [0, sg.total).
template <int KY, int DKM>
__device__ __forceinline__ void na3d_bwd_dkv_strip_body(const Na3dBwdParams& p, const BwdStrips& sg, char* lds, int id) {
#if defined(__HIP_DEVICE_COMPILE__)
  using namespace dkvs;
  constexpr int NS = (TY + KY - 1) / RPS;
  constexpr int KR = KY / 2;
  static_assert(TY + KY - 1 == NS * RPS, "one tile starts per row group");

  // ---- work unit: x box fastest, then key slice z, chunk, head, batch ----
  int t = xcd_tile_order(sg.total, id);
  const int xb = t % sg.nxt;
  t /= sg.nxt;
  const int z = t % p.Z;
  t /= p.Z;
  const int ch = t % sg.nch;
  t /= sg.nch;
  const int h = t % p.H;
  const int b = t / p.H;
  const int ys = sg.y0 + ch * sg.cty * TY;  // key rows [ys, ye)
  const int ye = min(ys + sg.cty * TY, sg.y1);
  const int x0 = xb * (NWX * TX);
  if (ys >= ye) return;  // uniform over the workgroup
  const int NT = (ye - ys + TY - 1) / TY;
  const int S = ys - KR;            // first query row of tile 0's inverse window
  const int NR = ye - ys + 2 * KR;  // query rows the strip streams
  const int NG = (NR + RPS - 1) / RPS;
  const int kz = p.ker[0], kx = p.ker[2];
  int zq0, nzq, QX0, wq0, cnt;
  axis_inv(z, p.Z, kz, 1, zq0, nzq);            // query slices whose windows hold slice z
  axis_inv(min(x0, p.X - 1), p.X, kx, 1, QX0, cnt);  // first staged query column

  const int tid = (int)__builtin_amdgcn_workitem_id_x();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n16 = lane & 15;
  const int g = lane >> 4;
  const int trow = n16 / TX;  // this lane's key row within a tile
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

  // ---- x geometry: the wave's 16-query block and this lane's key ----
  const int xw0 = x0 + wave * TX;
  axis_inv(min(xw0, p.X - 1), p.X, kx, 1, wq0, cnt);
  const int qb = wq0 - QX0;  // the wave's block in the staged row (<= LW - 16, checked by the host)
  const int kxl = xw0 + n16 % TX;
  f32x4 xbias;  // 0 or -inf: query 4g + i of the block holds / misses the lane's key in its x window
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int qx = QX0 + qb + 4 * g + i;
    const int sx = win_start(min(qx, p.X - 1), p.X, kx);
    xbias[i] = qx < p.X && kxl >= sx && kxl < sx + kx ? 0.f : -INFINITY;
  }
  const float c2 = p.scale * 1.4426950408889634f;

  // ---- tensor geometry (contiguous [B, Z, Y, X, H, D]) ----
  const int64_t colb = (int64_t)p.H * D * 2;
  const int64_t rowb = (int64_t)p.X * colb;
  const int64_t zb = (int64_t)p.Y * rowb;
  const int64_t slice = ((int64_t)b * p.Z + z) * zb + (int64_t)h * D * 2;  // (b, z, h) of the keys

  // ---- ring: Q rows (waves 0-1) or dO rows (waves 2-3), then one statistics row per wave ----
  const bool owave = wave >= 2;
  uint32_t doff[LPT];
#pragma unroll
  for (int i = 0; i < LPT; ++i) {
    const int f = ((wave & 1) * LPT + i) * KPK + lane / CPK;
    const int row = f / LW, col = f % LW;
    const int c = (lane % CPK) ^ (f & 7);
    doff[i] = QX0 + col < p.X ? (uint32_t)(row * rowb + (int64_t)(QX0 + col) * colb + 16 * c) : OOB;
  }
  const char* qseg = (const char*)(owave ? p.dout : p.q) + ((int64_t)b * p.Z + zq0) * zb + (int64_t)h * D * 2 +
                     (int64_t)S * rowb;
  // statistics: wave w copies row (w & 1) of lse (w < 2) or of D (w >= 2)
  const int64_t srow = (int64_t)p.X * p.H, sz = (int64_t)p.Y * srow;
  const float* sseg = (owave ? p.dsum : p.lse) + ((int64_t)b * p.Z + zq0) * sz + (int64_t)S * srow + h;
  const uint32_t soff = lane < LW && QX0 + lane < p.X ? (uint32_t)((QX0 + lane) * p.H * 4) : OOB;
  int cz = 0, cp = 0;
  uint32_t issue_off = 0;
  auto issue = [&]() {
    const int nrow = min(max(NR - RPS * cp, 0), RPS);
    const u32x4 rs = make_rsrc(qseg + (int64_t)cp * RPS * rowb + (int64_t)cz * zb, (uint32_t)(nrow * rowb));
    const uint32_t m0 = lds_base + issue_off + (uint32_t)wave * (LPT * 1024);
#pragma unroll
    for (int i = 0; i < LPT; ++i) dma_row16(rs, m0 + i * 1024, doff[i]);
    if (DKM || !owave) {  // dV needs no D
      const int r = wave & 1;
      const u32x4 rst = make_rsrc(sseg + (int64_t)(cp * RPS + r) * srow + (int64_t)cz * sz,
                                  r < nrow ? (uint32_t)(srow * 4) : 0u);
      dma_dword(rst, lds_base + issue_off + 2 * RPS * RB + (uint32_t)wave * SB, soff);
    }
    issue_off = issue_off + STAGE_B == RING_B ? 0 : issue_off + STAGE_B;
    if (++cz == nzq) {
      cz = 0;
      ++cp;
    }
  };

  // ---- K (and V) of a key tile: one (b, z, h) slice ----
  const uint32_t krec = (uint32_t)(zb - (int64_t)h * D * 2);
  const u32x4 rk = make_rsrc((const char*)p.k + slice, krec);
  const u32x4 rv = make_rsrc((const char*)p.v + slice, krec);
  auto dma_tile = [&](int j, uint32_t off) {
    const int yt0 = ys + TY * j;
    const uint32_t m0 = lds_base + off + (uint32_t)wave * TWB;
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      const int n = lane / CPK + i * (64 / CPK);
      const int ky = min(yt0 + n / TX, ye - 1), cx = min(xw0 + n % TX, p.X - 1);
      const uint32_t o = (uint32_t)(ky * rowb + cx * colb) + 16 * (lane % CPK);
      dma_row16(rk, m0 + i * 1024, o);
      if (DKM) dma_row16(rv, m0 + KWB + i * 1024, o);
    }
  };

  // ---- LDS read offsets within row 0 of a stage (row r adds r * RB) ----
  uint32_t aoff[KS], toff[DB];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int col = qb + n16;
    aoff[ks] = (col * D + 8 * ((4 * ks + g) ^ (col & 7))) * 2;
  }
  {
    const int colv = qb + 4 * g + (n16 >> 2), dq = n16 & 3;
#pragma unroll
    for (int db = 0; db < DB; ++db)
      toff[db] = (colv * D + 8 * ((2 * db + (dq >> 1)) ^ (colv & 7)) + 4 * (dq & 1)) * 2;
  }
  const uint32_t stoff = 2 * RPS * RB + 4 * (qb + 4 * g);  // this lane's 4 queries in a statistics row

  // ---- tile slots ----
  bf16x8 kreg[NS][KS], vreg[NS][KS];
  f32x4 acc[NS][DB];
  const bool ylo = trow > 0;  // first group: query row 0 masked for key row 1
  const bool yhi = trow < 1;  // last group: query row 1 masked for key row 0

  auto start_tile = [&](int k, uint32_t off) {
    const char* kb = lds + off + wave * TWB;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kreg[k][ks] = *(const bf16x8*)(kb + n16 * D * 2 + (4 * ks + g) * 16);
#pragma unroll
      for (int e = 0; e < 8; ++e) kreg[k][ks][e] = (bf16)((float)kreg[k][ks][e] * c2);
      if (DKM) vreg[k][ks] = *(const bf16x8*)(kb + KWB + n16 * D * 2 + (4 * ks + g) * 16);
    }
#pragma unroll
    for (int db = 0; db < DB; ++db) acc[k][db] = (f32x4){0.f, 0.f, 0.f, 0.f};
  };
  char* outb = (char*)(DKM ? p.dk : p.dv) + slice + 8 * g;
  const float oscale = DKM ? p.scale : 1.f;
  auto finish_tile = [&](int k, int j) {
    const int ky = ys + TY * j + trow;
    if (ky < ye && kxl < p.X) {
      char* op = outb + (int64_t)ky * rowb + (int64_t)kxl * colb;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const u32x2 w = {pack_bf16x2(acc[k][db][0] * oscale, acc[k][db][1] * oscale),
                         pack_bf16x2(acc[k][db][2] * oscale, acc[k][db][3] * oscale)};
        *(u32x2*)(op + 32 * db) = w;
      }
    }
  };

  auto stage_math = [&](auto cst, auto act, const char* st) {
    constexpr int C = decltype(cst)::value;
    constexpr int ACT = decltype(act)::value;
    bf16x8 qa[RPS][KS], oa[RPS][KS], tr[DB];
    float lsq[RPS][4], dsq[RPS][4];
#pragma unroll
    for (int r = 0; r < RPS; ++r) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        qa[r][ks] = *(const bf16x8*)(st + r * RB + aoff[ks]);
        if (DKM) oa[r][ks] = *(const bf16x8*)(st + (RPS + r) * RB + aoff[ks]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lsq[r][i] = *(const float*)(st + stoff + r * SB + 4 * i);
        if (DKM) dsq[r][i] = *(const float*)(st + stoff + (RPS + r) * SB + 4 * i);
      }
    }
    // dO^T (dV) or Q^T (dK) over the row pair
    const int tbase = DKM ? 0 : RPS * RB;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, st + tbase + toff[db]));
      const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, st + tbase + RB + toff[db]));
      tr[db] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
    static_for<NS>([&](auto ttc) {
      constexpr int tt = decltype(ttc)::value;  // 0: the tile's first group, 1: its last
      constexpr int k = (C + tt) % NS;
      if constexpr ((ACT >> k) & 1) {
        float pv[RPS][4];
#pragma unroll
        for (int r = 0; r < RPS; ++r) {
          f32x4 sc = xbias;
#pragma unroll
          for (int ks = 0; ks < KS; ++ks)
            sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[r][ks], kreg[k][ks], sc, 0, 0, 0);
          const bool masked = (tt == 0 && r == 0 && ylo) || (tt == 1 && r == 1 && yhi);
          if constexpr (DKM) {
            f32x4 dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
              dp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(oa[r][ks], vreg[k][ks], dp, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e)
              pv[r][e] = masked ? 0.f : __builtin_amdgcn_exp2f(sc[e] - lsq[r][e]) * (dp[e] - dsq[r][e]);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) pv[r][e] = masked ? 0.f : __builtin_amdgcn_exp2f(sc[e] - lsq[r][e]);
          }
        }
        const bf16x8 pb = __builtin_bit_cast(
            bf16x8, ((u32x4){pack_bf16x2(pv[0][0], pv[0][1]), pack_bf16x2(pv[0][2], pv[0][3]),
                             pack_bf16x2(pv[1][0], pv[1][1]), pack_bf16x2(pv[1][2], pv[1][3])}));
#pragma unroll
        for (int db = 0; db < DB; ++db)
          acc[k][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tr[db], pb, acc[k][db], 0, 0, 0);
      }
    });
  };

  // Tile 0's keys are staged through the ring before the ring starts.
  dma_tile(0, 0);
  wait_vmcnt(0);
  start_tile(0, 0);
  wait_lgkm0();
  lds_barrier();
#pragma unroll
  for (int s = 0; s < NBUF - 1; ++s) issue();

  uint32_t cur_off = 0;
  auto group = [&](auto cst, auto act, int gr) {
    constexpr int C = decltype(cst)::value;
    for (int zc = 0; zc < nzq; ++zc) {
      const bool starting = zc == 0 && gr > 0 && gr < NT;
      if (starting)
        wait_vmcnt(0);  // the tile's key copies as well
      else
        wait_vmcnt((NBUF - 2) * (LPT + 1));
      lds_barrier();
      issue();
      if (starting) start_tile(C, (uint32_t)RING_B);
      if (zc == 1 && gr + 1 < NT) dma_tile(gr + 1, (uint32_t)RING_B);
      stage_math(cst, act, lds + cur_off);
      cur_off = cur_off + STAGE_B == RING_B ? 0 : cur_off + STAGE_B;
    }
    const int jf = gr - (NS - 1);
    if (jf >= 0 && jf < NT) finish_tile((C + 1) % NS, jf);
  };
  using ALL = std::integral_constant<int, (1 << NS) - 1>;
  static_for<NS - 1>([&](auto ig) {
    constexpr int G = decltype(ig)::value;
    group(std::integral_constant<int, G>{}, std::integral_constant<int, (1 << (G + 1)) - 1>{}, G);
  });
  for (int gr = NS - 1;; gr += NS) {  // NG = NT + NS - 1 >= NS
    bool done = false;
    static_for<NS>([&](auto ii) {
      constexpr int I = decltype(ii)::value;
      if (!done) {
        group(std::integral_constant<int, (NS - 1 + I) % NS>{}, ALL{}, gr + I);
        done = gr + I + 1 >= NG;
      }
    });
    if (done) break;
  }
  wait_vmcnt(0);
#endif
}


template <int KY>
__global__ __launch_bounds__(256, 2) void na3d_bwd_dq_strip_kernel(Na3dBwdParams p, BwdStrips sg) {
  __shared__ __attribute__((aligned(1024))) char lds[dqs::LDS_B];
  na3d_bwd_dq_strip_body<KY>(p, sg, lds, (int)__builtin_amdgcn_workgroup_id_x());
}

// The backward's small-window launch: dq, dV and dK on strips and the clamped
// edge rows of each on the tile walks, as one grid (the parts are independent:
// each writes its own rows of dq, dk or dv).  Part k takes workgroup ids
// [base[k], base[k + 1]) (each part padded to a multiple of 8, so it keeps its
// XCD-aware order); the strip parts come first, the edge workgroups fill their
// tail (measured: the edge parts first is 2.5% slower).  Edge parts: dq top /
// bottom (rows [0, sq.y0) and [sq.y1, Y): ky/2 rows, on workgroups of one
// 4-row tile, BWD_DQE_NT), dk/dv top / bottom (rows [0, skv.y0) and
// [skv.y1, Y): 2 (ky/2) + 1 rows, on workgroups of two 4-row tiles,
// BWD_DKVE_NT).  Measured against 8-row workgroups for both: configs[1]
// 0.454 -> 0.428 ms (4-row dk/dv edges as well: 0.445 ms).
constexpr int BWD_DQE_NT = 1;
constexpr int BWD_DKVE_NT = 2;
struct BwdParts {
  int base[8];   // dq strips, dV strips, dK strips, dq top, dq bottom, dkv top, dkv bottom, end
  int nyt[4];    // tile rows of the four edge parts
};

template <int KY>
__global__ __launch_bounds__(256, 2) void na3d_bwd_small_fused_kernel(Na3dBwdParams p, BwdStrips sq, BwdStrips skv,
                                                                       BwdParts parts) {
  constexpr int LB = dqs::LDS_B > dkvs::LDS_B ? dqs::LDS_B : dkvs::LDS_B;
  static_assert(LB >= dql::NBUF * dql::STAGE && LB >= dkvl::NBUF * dkvl::STAGE, "one LDS buffer for every part");
  __shared__ __attribute__((aligned(1024))) char lds[LB];
  const int id = (int)__builtin_amdgcn_workgroup_id_x();
  int k = 0;
  while (k < 7 && id >= parts.base[k + 1]) ++k;  // uniform
  const int w = id - parts.base[k];
  switch (k) {
    case 0:
      if (w < sq.total) na3d_bwd_dq_strip_body<KY>(p, sq, lds, w);
      break;
    case 1:
      if (w < skv.total) na3d_bwd_dkv_strip_body<KY, 0>(p, skv, lds, w);
      break;
    case 2:
      if (w < skv.total) na3d_bwd_dkv_strip_body<KY, 1>(p, skv, lds, w);
      break;
    default: {
      const int e = k - 3;  // 0, 1: dq top / bottom; 2, 3: dk/dv top / bottom
      const BwdStrips& s = e < 2 ? sq : skv;
      Na3dBwdParams pe = p;
      pe.qy0 = (e & 1) ? s.y1 : 0;
      pe.qny = (e & 1) ? p.Y - s.y1 : s.y0;
      const int n = p.B * p.H * p.Z * parts.nyt[e] * p.nxt;
      if (w < n) {
        if (e < 2)
          na3d_bwd_dq_lds_body<BWD_DQE_NT>(pe, parts.nyt[e], lds, w);
        else
          na3d_bwd_dkv_lds_body<BWD_DKVE_NT>(pe, parts.nyt[e], lds, w);
      }
    }
  }
}

// D_i = dO_i . O_i alone, for a backward given the forward's log-sum-exp:
// LPR lanes per (token, head) row, 16 bytes of dO and of O each, closed by
// xor shuffles.
template <typename T, int D>
__global__ __launch_bounds__(256) void na3d_bwd_dsum_kernel(Na3dBwdParams p, int64_t rows) {
  constexpr int EPL = 16 / (int)sizeof(T), LPR = D / EPL;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = idx / LPR;
  const int c = (int)(idx % LPR);
  float s = 0.f;
  if (row < rows) {
    float a[EPL], o[EPL];
    load_dims<T, EPL>((const T*)p.dout + row * D + c * EPL, a);
    load_dims<T, EPL>((const T*)p.o + row * D + c * EPL, o);
#pragma unroll
    for (int e = 0; e < EPL; ++e) s = fmaf(a[e], o[e], s);
  }
  for (int sh = 1; sh < LPR; sh <<= 1) s += __shfl_xor(s, sh);
  if (row < rows && c == 0) p.dsum[row] = s;
}

// The MFMA kernels: dilation 1, kx <= 13 (a 4-column tile's x union fits one 16-key block).
// The LDS kernels' copies address one (b, z, y) row of a tensor with 32-bit
// offsets (X * H * D bf16), the statistics two rows apart (one z-slice).
static bool mfma_ok(const Na3dBwdParams& p) {
  const int64_t row = (int64_t)p.X * p.H;
  return p.dil[0] == 1 && p.dil[1] == 1 && p.dil[2] == 1 && p.ker[2] <= 13 && row * 64 * 2 < (int64_t)OOB &&
         ((int64_t)p.Y + 1) * row * 4 < (int64_t)OOB && !std::getenv("STRATA_HIP_NA3D_BWD_VALU");
}

// dq on strips (na3d_bwd_dq_strip_kernel): kx <= 9, ky in {3, 5, 7}, kz >= 2, at
// least two unclamped rows, and one (b, z) slice of Q / dO / statistics within
// 31-bit offsets.  STRATA_HIP_NA3D_BWD_NO_STRIPS=1 switches the path off.
static bool dq_strip_fits(const Na3dBwdParams& p) {
  const int ky = p.ker[1];
  if (p.ker[0] < 2 || p.ker[2] > 9 || (ky != 3 && ky != 5 && ky != 7)) return false;  // ky = 9 would spill
  if (p.Y - 2 * (ky / 2) < 2) return false;
  if ((int64_t)p.Y * p.X * p.H * 64 * 2 >= 0x7fffffffLL) return false;
  return !std::getenv("STRATA_HIP_NA3D_BWD_NO_STRIPS");
}

// Strip work units: (b, h, z, 32-column box), the strip rows cut into chunks
// only while that leaves fewer than one round of two workgroups per CU.
static bool make_bwd_strips(const Na3dBwdParams& p, int y0, int y1, BwdStrips& sg) {
  sg.y0 = y0;
  sg.y1 = y1;
  sg.nxt = (p.X + 31) / 32;
  const int nty = (sg.y1 - sg.y0 + 1) / 2;
  const int64_t strips = (int64_t)p.B * p.H * p.Z * sg.nxt;
  int nch = 1;
  while (strips * nch < 512 && nch < nty) ++nch;
  sg.cty = (nty + nch - 1) / nch;
  sg.nch = (nty + sg.cty - 1) / sg.cty;
  const int64_t total = strips * sg.nch;
  if (total <= 0 || total > 0x7fffffff) return false;
  sg.total = (int)total;
  return true;
}

// dK / dV on strips (na3d_bwd_dkv_strip_kernel): the dq conditions, kz >= 3 (every
// key slice then lies in at least two query slices' windows), at least two key rows
// that no clamped query window reaches, and along x every wave's query block (16
// columns from the first query holding its first key column) and every
// workgroup's staged row (40 columns) covering their keys' inverse windows.
static bool dkv_strip_fits(const Na3dBwdParams& p) {
  if (!dq_strip_fits(p) || p.ker[0] < 3) return false;
  const int kr = p.ker[1] / 2, kx = p.ker[2];
  if (p.Y - 2 * (2 * kr + 1) < 2) return false;
  int f0, n0, f1, n1;
  for (int x0 = 0; x0 < p.X; x0 += 8) {
    axis_inv(x0, p.X, kx, 1, f0, n0);
    axis_inv(std::min(x0 + 7, p.X - 1), p.X, kx, 1, f1, n1);
    if (f1 + n1 - f0 > 16) return false;
  }
  for (int x0 = 0; x0 < p.X; x0 += 32) {
    axis_inv(x0, p.X, kx, 1, f0, n0);
    axis_inv(std::min(x0 + 31, p.X - 1), p.X, kx, 1, f1, n1);
    if (f1 + n1 - f0 > 40) return false;
    for (int w = 1; w < 4 && x0 + 8 * w < p.X; ++w) {
      int fw, nw;
      axis_inv(x0 + 8 * w, p.X, kx, 1, fw, nw);
      if (fw - f0 + 16 > 40) return false;
    }
  }
  return true;
}

static void launch_dq_strips(const Na3dBwdParams& p, const BwdStrips& sg, hipStream_t st) {
  const dim3 grid((unsigned)sg.total), block(256);
  switch (p.ker[1]) {
    case 3: hipLaunchKernelGGL(na3d_bwd_dq_strip_kernel<3>, grid, block, 0, st, p, sg); break;
    case 5: hipLaunchKernelGGL(na3d_bwd_dq_strip_kernel<5>, grid, block, 0, st, p, sg); break;
    default: hipLaunchKernelGGL(na3d_bwd_dq_strip_kernel<7>, grid, block, 0, st, p, sg); break;
  }
}

template <typename T, int D>
static int launch_bwd(const Na3dBwdParams& p, hipStream_t st) {
  const int64_t blocks = (int64_t)p.B * p.H * p.Z * p.nyt * p.nxt;
  if (blocks == 0) return STRATA_HIP_OK;
  if (blocks > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "na3d_bwd: problem too large for one launch");
  const dim3 grid((unsigned)blocks), block(256);
  if (p.lse_given) {
    constexpr int LPR = D * (int)sizeof(T) / 16;
    const int64_t rows = (int64_t)p.B * p.Z * p.Y * p.X * p.H;
    hipLaunchKernelGGL((na3d_bwd_dsum_kernel<T, D>), dim3((unsigned)((rows * LPR + 255) / 256)), block, 0, st, p,
                       rows);
  } else if (sizeof(T) == 2 && D == 64 && mfma_ok(p)) {
    hipLaunchKernelGGL(na3d_bwd_prep_mfma_kernel, grid, block, 0, st, p);
  } else {
    hipLaunchKernelGGL((na3d_bwd_prep_kernel<T, D>), grid, block, 0, st, p);
  }
  // LDS kernels: workgroups of 4 * NT rows
  constexpr int NT = NA3D_BWD_NT;
  const int nyt_lds = (p.Y + 4 * NT - 1) / (4 * NT);
  const dim3 grid_lds((unsigned)((int64_t)p.B * p.H * p.Z * nyt_lds * p.nxt));
  if (sizeof(T) == 2 && D == 64 && mfma_ok(p)) {
    // dq, dV and dK on strips with every clamped edge in one launch
    BwdStrips sq, skv;
    const int kr = p.ker[1] / 2, ek = 2 * kr + 1;
    if (dkv_strip_fits(p) && make_bwd_strips(p, kr, p.Y - kr, sq) && make_bwd_strips(p, ek, p.Y - ek, skv)) {
      static_assert(NT == NA3D_BWD_NT, "edge parts: workgroups of 4 NT rows");
      BwdParts parts;
      const int rows[4] = {sq.y0, p.Y - sq.y1, skv.y0, p.Y - skv.y1};
      int64_t count[7] = {sq.total, skv.total, skv.total, 0, 0, 0, 0};
      for (int e = 0; e < 4; ++e) {
        const int ert = 4 * (e < 2 ? BWD_DQE_NT : BWD_DKVE_NT);  // rows per edge workgroup
        parts.nyt[e] = (rows[e] + ert - 1) / ert;
        count[3 + e] = (int64_t)p.B * p.H * p.Z * parts.nyt[e] * p.nxt;
      }
      int64_t base = 0;
      for (int k = 0; k < 7; ++k) {
        if (base > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "na3d_bwd: problem too large for one launch");
        parts.base[k] = (int)base;
        base += (count[k] + 7) / 8 * 8;
      }
      if (base > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "na3d_bwd: problem too large for one launch");
      parts.base[7] = (int)base;
      if (p.ker[1] == 3)
        hipLaunchKernelGGL(na3d_bwd_small_fused_kernel<3>, dim3((unsigned)base), block, 0, st, p, sq, skv, parts);
      else if (p.ker[1] == 5)
        hipLaunchKernelGGL(na3d_bwd_small_fused_kernel<5>, dim3((unsigned)base), block, 0, st, p, sq, skv, parts);
      else
        hipLaunchKernelGGL(na3d_bwd_small_fused_kernel<7>, dim3((unsigned)base), block, 0, st, p, sq, skv, parts);
      return check_launch("na3d_bwd kernels");
    }
  }
  if (sizeof(T) == 2 && D == 64 && mfma_ok(p)) {
    BwdStrips sg;
    const int kr = p.ker[1] / 2;
    if (dq_strip_fits(p) && make_bwd_strips(p, kr, p.Y - kr, sg)) {
      // the unclamped rows on strips, the clamped ones at each y edge on the tile walk
      static_assert(NT == 2, "edge rows: workgroups of 8 rows");
      launch_dq_strips(p, sg, st);
      Na3dBwdParams e = p;
      for (int side = 0; side < 2; ++side) {
        e.qy0 = side ? sg.y1 : 0;
        e.qny = side ? p.Y - sg.y1 : sg.y0;
        const int nyt_e = (e.qny + 4 * NT - 1) / (4 * NT);
        const int64_t ge = (int64_t)p.B * p.H * p.Z * nyt_e * p.nxt;
        if (ge > 0) hipLaunchKernelGGL(na3d_bwd_dq_lds_kernel<NT>, dim3((unsigned)ge), block, 0, st, e, nyt_e);
      }
    } else {
      hipLaunchKernelGGL(na3d_bwd_dq_lds_kernel<NT>, grid_lds, block, 0, st, p, nyt_lds);
    }
  } else {
    hipLaunchKernelGGL((na3d_bwd_dq_kernel<T, D>), grid, block, 0, st, p);
  }
  if (sizeof(T) == 2 && D == 64 && mfma_ok(p))
    hipLaunchKernelGGL(na3d_bwd_dkv_lds_kernel<NT>, grid_lds, block, 0, st, p, nyt_lds);
  else
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

// Scratch of strata_hip_na3d_bwd_noalloc: the per-query log-sum-exp and
// rowsum(dout * out) of one call, for at most NA3D_BWD_SCRATCH_TOKENS
// (query, head) pairs (16 MiB).  Every device the library runs on holds its own
// copy until the process ends; host code reaches it only through the address
// hipGetSymbolAddress returns for that device (the array's name is a host-side
// stand-in, not a device address).  Calls on one device share it: two calls
// that overlap in time on one device race.
constexpr int64_t NA3D_BWD_SCRATCH_TOKENS = int64_t(1) << 21;
static __device__ __align__(256) float scratch[2 * NA3D_BWD_SCRATCH_TOKENS];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch[MAX_DEVICES] = {};

// The current device's copy of `scratch`, looked up once per device.
int scratch_for_current_device(float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return fail(STRATA_HIP_ELAUNCH, "na3d_bwd_noalloc: no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(STRATA_HIP_ELAUNCH, std::string("na3d_bwd_noalloc: hipGetSymbolAddress(scratch): ") +
                                          hipGetErrorString(e));
    g_scratch[dev] = (float*)ptr;
  }
  *out = g_scratch[dev];
  return STRATA_HIP_OK;
}
}  // namespace

// Argument checks and the launch shared by both entry points; `workspace` is
// the caller's buffer or this device's scratch.
static int na3d_bwd_run(const strata_hip_na3d_bwd_args* a, float* workspace, void* stream);

extern "C" int strata_hip_na3d_bwd(const strata_hip_na3d_bwd_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "na3d_bwd: null args");
  return na3d_bwd_run(a, a->workspace, stream);
}

extern "C" int strata_hip_na3d_bwd_noalloc(const strata_hip_na3d_bwd_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "na3d_bwd_noalloc: null args");
  if (a->workspace)
    return fail(STRATA_HIP_EINVAL, "na3d_bwd_noalloc: workspace must be NULL (the library's scratch is used)");
  if (a->batch < 0 || a->heads <= 0 || a->grid[0] <= 0 || a->grid[1] <= 0 || a->grid[2] <= 0)
    return fail(STRATA_HIP_EINVAL, "na3d_bwd_noalloc: bad batch/heads/grid");
  const int64_t tokens = (int64_t)a->batch * a->grid[0] * a->grid[1] * a->grid[2] * a->heads;
  if (tokens > NA3D_BWD_SCRATCH_TOKENS)
    return fail(STRATA_HIP_EUNSUPPORTED,
                "na3d_bwd_noalloc: B*Z*Y*X*H = " + std::to_string(tokens) + " exceeds the scratch maximum of " +
                    std::to_string(NA3D_BWD_SCRATCH_TOKENS) + " (query, head) pairs; use strata_hip_na3d_bwd");
  if (tokens == 0) return na3d_bwd_run(a, nullptr, stream);
  float* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc != STRATA_HIP_OK) return rc;
  return na3d_bwd_run(a, ws, stream);
}

static int na3d_bwd_run(const strata_hip_na3d_bwd_args* a, float* workspace, void* stream) {
  if (a->dtype != STRATA_HIP_F32 && a->dtype != STRATA_HIP_BF16)
    return fail(STRATA_HIP_EINVAL, "na3d_bwd: dtype must be f32 or bf16");
  if (a->batch < 0 || a->heads <= 0 || a->head_dim <= 0)
    return fail(STRATA_HIP_EINVAL, "na3d_bwd: bad batch/heads/head_dim");
  static const char* axis = "zyx";
  for (int i = 0; i < 3; ++i) {
    const int L = a->grid[i], k = a->kernel[i], d = a->dilation[i];
    if (L <= 0) return fail(STRATA_HIP_EINVAL, std::string("na3d_bwd: grid size must be positive on axis ") + axis[i]);
    // Odd, or the whole undilated axis (as the forward; axis_inv then spans the axis).
    if (k <= 0 || ((k % 2) == 0 && !(k == L && d == 1)))
      return fail(STRATA_HIP_EINVAL,
                  std::string("na3d_bwd: kernel size must be odd and positive (or the whole axis) on axis ") + axis[i]);
    if (d <= 0) return fail(STRATA_HIP_EINVAL, std::string("na3d_bwd: dilation must be positive on axis ") + axis[i]);
    if ((int64_t)d * k > L)
      return fail(STRATA_HIP_EINVAL, std::string("na3d_bwd: dilation * kernel exceeds the grid on axis ") + axis[i]);
  }
  if (a->batch == 0) return STRATA_HIP_OK;
  const void* ptrs[] = {a->q, a->k, a->v, a->out, a->dout, a->dq, a->dk, a->dv, workspace};
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
  p.lse = workspace;
  p.dsum = workspace + tokens;
  if (a->lse) {  // the forward's statistics: prep reduces to D_i
    if ((uintptr_t)a->lse & 3u) return fail(STRATA_HIP_EINVAL, "na3d_bwd: lse must be 4-byte aligned");
    if (tokens * (a->head_dim * (a->dtype == STRATA_HIP_BF16 ? 2 : 4) / 16) / 256 + 1 > 0x7fffffff)
      return fail(STRATA_HIP_EUNSUPPORTED, "na3d_bwd: problem too large for one launch");
    p.lse = const_cast<float*>(a->lse);
    p.lse_given = 1;
  }
  p.nyt = (p.Y + 3) / 4;
  p.nxt = (p.X + 15) / 16;
  p.qy0 = 0;
  p.qny = p.Y;
  hipStream_t st = (hipStream_t)stream;
  return a->dtype == STRATA_HIP_BF16 ? launch_bwd_t<bf16>(p, a->head_dim, st) : launch_bwd_t<float>(p, a->head_dim, st);
}
