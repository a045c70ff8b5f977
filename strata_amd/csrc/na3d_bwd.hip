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
// Three kernels, each a wave per 4 x 4 tile of tokens.  bf16 with head_dim 64
// and dilation 1 (the training shapes) runs MFMA versions (below); the general
// VALU versions (4 lanes per token, D/4 head dims per lane, dot products closed
// by two xor shuffles) take everything else:
//   prep: per query, log2-sum-exp of its scores (recomputed, unless the caller
//         passes the forward's, strata_hip_na3d_fwd's lse output: then only
//         D_i) and D_i, into a caller-provided fp32 workspace;
//   dq:   per query, a walk over its window;
//   dkv:  per key, a walk over its inverse window {i : j in W(i)}, which per
//         axis is an interval (window starts are non-decreasing in i):
//         lo = 0 if j <= k - 1 else j - k + 1 + k/2,  hi = Lg - 1 if j >= Lg - k else j + k/2
//         (sub-grid coordinates of the dilation residue class).
// Scores run in log2 units (q pre-scaled by scale * log2 e), fp32 throughout;
// the neighbouring tokens of a tile share most of their window, so their
// K/V (or Q/dO) reads hit in L1/L2.
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

// The token of in-tile index t (row t >> 2, column t & 3) of this lane's wave.
__device__ __forceinline__ Tok token_at(const Na3dBwdParams& p, int t) {
  int w = (int)blockIdx.x;
  const int xb = w % p.nxt;
  w /= p.nxt;
  const int yt = w % p.nyt;
  w /= p.nyt;
  const int z = w % p.Z;
  w /= p.Z;
  const int h = w % p.H;
  const int b = w / p.H;
  const int wave = (int)threadIdx.x >> 6;
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

// ---------------------------------------------------------------------------
// MFMA dq for bf16, head_dim 64, dilation 1 (the training shapes): a wave per
// 4 x 4 query tile walks its window union a (z, row pair) at a time.  Per row
// pair (32 keys of one 16-key x block): S^T = K Q^T and dP^T = V dO^T on
// v_mfma_f32_16x16x32_bf16 (keys on M, queries on N, both straight from
// global memory), dS^T = P^T (dP^T - D) in registers, and dQ^T += K^T dS^T
// with K^T read back transposed (ds_read_b64_tr_b16) from the two K rows the
// wave has just written to its own 4 KiB of LDS.  Masks: a per-lane bias of
// 0 / -inf per key for the x window and per row for the y window (the z
// window is the wave's for every query).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void na3d_bwd_dq_mfma_kernel(Na3dBwdParams p) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int D = 64, KS = 2, DB = 4, RBW = 16 * D * 2;  // bytes of one 16-key row in LDS
  __shared__ __attribute__((aligned(16))) char lds[4 * 2 * RBW];
  const int tid = (int)threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, n16 = lane & 15, g = lane >> 4;
  const Tok t = token_at(p, n16);  // MFMA column n16 = the lane's query
  char* wl = lds + wave * 2 * RBW;
  const float c2 = p.scale * 1.4426950408889634f;
  const int kz = p.ker[0], ky = p.ker[1], kx = p.ker[2];

  // this lane's query: n16 = (row, column) of the wave's 4 x 4 tile (as token_of)
  const int64_t qi = tok_index(p, t.b, t.z, t.y, t.x, t.h);
  bf16x8 qreg[KS], doreg[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qreg[ks] = *(const bf16x8*)((const bf16*)p.q + qi * D + 8 * (4 * ks + g));
    doreg[ks] = *(const bf16x8*)((const bf16*)p.dout + qi * D + 8 * (4 * ks + g));
#pragma unroll
    for (int e = 0; e < 8; ++e) qreg[ks][e] = (bf16)((float)qreg[ks][e] * c2);
  }
  const float lse = p.lse[qi], dsum = p.dsum[qi];

  // the wave's key block: 16 keys from the window start of its first column
  const int xw0 = min(((int)blockIdx.x % p.nxt) * 16 + wave * 4, p.X - 1);
  const int X0 = win_start(xw0, p.X, kx);
  const int sx = win_start(t.x, p.X, kx);
  f32x4 xb, ninf = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = X0 + 4 * g + i;
    xb[i] = (key >= sx && key < sx + kx) ? 0.f : -INFINITY;
  }
  const int kxl = min(X0 + n16, p.X - 1);  // key column this lane loads (clamped)
  // rows: the union of the tile rows' windows
  const int ty0 = ((int)(blockIdx.x / p.nxt) % p.nyt) * 4;
  const int Yu0 = win_start(min(ty0, p.Y - 1), p.Y, ky);
  const int NR = win_start(min(ty0 + 3, p.Y - 1), p.Y, ky) + ky - Yu0;
  const int sy = win_start(t.y, p.Y, ky);
  const int sz = win_start(t.z, p.Z, kz);
  // V^T-style transposed read offsets within a row (as the forward's PV operand)
  uint32_t toff[DB];
  {
    const int keyv = 4 * g + (n16 >> 2), dq = n16 & 3;
#pragma unroll
    for (int db = 0; db < DB; ++db)
      toff[db] = (uint32_t)((keyv * D + 8 * ((2 * db + (dq >> 1)) ^ (keyv & 7)) + 4 * (dq & 1)) * 2);
  }
  f32x4 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = (f32x4){0.f, 0.f, 0.f, 0.f};

  for (int a0 = 0; a0 < kz; ++a0) {
    const int zk = sz + a0;
    for (int r0 = 0; r0 < NR; r0 += 2) {
      bf16x8 ak[2][KS], avn[2][KS];
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int yk = min(Yu0 + r0 + rr, p.Y - 1);
        const int64_t kj = tok_index(p, t.b, zk, yk, kxl, t.h);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          ak[rr][ks] = *(const bf16x8*)((const bf16*)p.k + kj * D + 8 * (4 * ks + g));
          avn[rr][ks] = *(const bf16x8*)((const bf16*)p.v + kj * D + 8 * (4 * ks + g));
        }
      }
      // K rows into this wave's LDS (swizzled 16-byte chunks) for the transposed read
#pragma unroll
      for (int rr = 0; rr < 2; ++rr)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          *(bf16x8*)(wl + rr * RBW + n16 * D * 2 + 16 * ((4 * ks + g) ^ (n16 & 7))) = ak[rr][ks];
      f32x4 sc[2], dp[2];
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int yk = Yu0 + r0 + rr;
        const bool rowin = r0 + rr < NR && yk >= sy && yk < sy + ky;
        sc[rr] = rowin ? xb : ninf;
        dp[rr] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          sc[rr] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak[rr][ks], qreg[ks], sc[rr], 0, 0, 0);
          dp[rr] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(avn[rr][ks], doreg[ks], dp[rr], 0, 0, 0);
        }
      }
      float ds[8];
#pragma unroll
      for (int rr = 0; rr < 2; ++rr)
#pragma unroll
        for (int i = 0; i < 4; ++i) ds[4 * rr + i] = exp2f(sc[rr][i] - lse) * (dp[rr][i] - dsum);
      const u32x4 pw = {pack_bf16x2(ds[0], ds[1]), pack_bf16x2(ds[2], ds[3]), pack_bf16x2(ds[4], ds[5]),
                        pack_bf16x2(ds[6], ds[7])};
      const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);
      wait_lds();  // this wave's K rows are in LDS
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, wl + toff[db]));
        const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, wl + RBW + toff[db]));
        acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), pb,
                                                          acc[db], 0, 0, 0);
      }
      wait_lds();  // the transposed reads are done before the next pair overwrites the rows
    }
  }
  if (t.valid) {
    char* op = (char*)p.dq + 2 * (qi * D) + 8 * g;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const u32x2 w = {pack_bf16x2(acc[db][0] * p.scale, acc[db][1] * p.scale),
                       pack_bf16x2(acc[db][2] * p.scale, acc[db][3] * p.scale)};
      *(u32x2*)(op + 32 * db) = w;
    }
  }
#endif
}

// ---------------------------------------------------------------------------
// MFMA prep for bf16, head_dim 64, dilation 1: the dq kernel's walk with the
// score MFMA only.  Each lane keeps a running maximum and sum over the 8 keys
// of its query it sees per row pair; the four lanes of a query (g = 0..3)
// merge them at the end.  D_i = dO_i . O_i on the same lanes.
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
// MFMA dk / dv for bf16, head_dim 64, dilation 1: a wave per 4 x 4 key tile
// walks the union of its keys' inverse windows in blocks of 16 queries (one
// (z, y) row, 16 consecutive x), two blocks at a time.  Per block: S = Q K^T
// and dP = dO V^T (queries on M straight from global memory, the tile's K / V
// held in registers as the N operand), P = 2^(S - lse), dS = P (dP - D); per
// pair: dV^T += dO^T P and dK^T += Q^T dS (K = the pair's 32 queries) with
// dO^T and Q^T read back transposed from the wave's own 8 KiB of LDS.  The
// membership mask (key j in the window of query i, per axis) is the C operand
// of the S MFMA.  Q is staged pre-scaled by scale * log2 e, so dK carries a
// factor ln 2 at the end.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void na3d_bwd_dkv_mfma_kernel(Na3dBwdParams p) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int D = 64, KS = 2, DB = 4, RBW = 16 * D * 2;
  __shared__ __attribute__((aligned(16))) char lds[4 * 4 * RBW];  // per wave: Q rows 0, 1; dO rows 0, 1
  const int tid = (int)threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, n16 = lane & 15, g = lane >> 4;
  const Tok t = token_at(p, n16);  // MFMA column n16 = the lane's key
  char* wl = lds + wave * 4 * RBW;
  const float c2 = p.scale * 1.4426950408889634f;
  const int kz = p.ker[0], ky = p.ker[1], kx = p.ker[2];

  const int64_t kj = tok_index(p, t.b, t.z, t.y, t.x, t.h);
  bf16x8 kreg[KS], vreg[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    kreg[ks] = *(const bf16x8*)((const bf16*)p.k + kj * D + 8 * (4 * ks + g));
    vreg[ks] = *(const bf16x8*)((const bf16*)p.v + kj * D + 8 * (4 * ks + g));
  }
  // the tile's keys: columns [kx0, kx1], rows [ky0, ky1] (clamped to the grid)
  const int kx0 = min(((int)blockIdx.x % p.nxt) * 16 + wave * 4, p.X - 1), kx1 = min(kx0 + 3, p.X - 1);
  const int ky0 = min(((int)(blockIdx.x / p.nxt) % p.nyt) * 4, p.Y - 1), ky1 = min(ky0 + 3, p.Y - 1);
  int f, n;
  axis_inv(kx0, p.X, kx, 1, f, n);
  const int QX0 = f;
  axis_inv(kx1, p.X, kx, 1, f, n);
  const int NXB = (f + n - QX0 + 15) / 16;  // 16-query blocks along x
  axis_inv(ky0, p.Y, ky, 1, f, n);
  const int QY0 = f;
  axis_inv(ky1, p.Y, ky, 1, f, n);
  const int NY = f + n - QY0;
  int QZ0, NZ;
  axis_inv(t.z, p.Z, kz, 1, QZ0, NZ);
  const int nb = NZ * NY * NXB;

  uint32_t toff[DB];  // transposed-read offsets within a 16-row block (as the forward's V^T)
  {
    const int keyv = 4 * g + (n16 >> 2), dq = n16 & 3;
#pragma unroll
    for (int db = 0; db < DB; ++db)
      toff[db] = (uint32_t)((keyv * D + 8 * ((2 * db + (dq >> 1)) ^ (keyv & 7)) + 4 * (dq & 1)) * 2);
  }
  f32x4 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dk[db] = dv[db] = (f32x4){0.f, 0.f, 0.f, 0.f};

  for (int bi = 0; bi < nb; bi += 2) {
    float pv[2][4], sv[2][4];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const int bj = bi + hb;
      const bool live = bj < nb;
      const int bjc = live ? bj : bi;
      const int xb = bjc % NXB, r = bjc / NXB;
      const int qy = QY0 + r % NY, qz = QZ0 + r / NY;
      const int qx = QX0 + 16 * xb + n16;  // the query this lane loads (A operand row n16)
      const int64_t qi = tok_index(p, t.b, qz, qy, min(qx, p.X - 1), t.h);
      bf16x8 qa[KS], da[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        qa[ks] = *(const bf16x8*)((const bf16*)p.q + qi * D + 8 * (4 * ks + g));
        da[ks] = *(const bf16x8*)((const bf16*)p.dout + qi * D + 8 * (4 * ks + g));
#pragma unroll
        for (int e = 0; e < 8; ++e) qa[ks][e] = (bf16)((float)qa[ks][e] * c2);
        *(bf16x8*)(wl + hb * RBW + n16 * D * 2 + 16 * ((4 * ks + g) ^ (n16 & 7))) = qa[ks];
        *(bf16x8*)(wl + (2 + hb) * RBW + n16 * D * 2 + 16 * ((4 * ks + g) ^ (n16 & 7))) = da[ks];
      }
      // mask: query rows 4g..4g+3 of the block against this lane's key
      const bool yz = live && t.y >= win_start(qy, p.Y, ky) && t.y < win_start(qy, p.Y, ky) + ky &&
                      t.z >= win_start(qz, p.Z, kz) && t.z < win_start(qz, p.Z, kz) + kz;
      f32x4 sc, dp = {0.f, 0.f, 0.f, 0.f};
      float lse[4], dsm[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qxi = QX0 + 16 * xb + 4 * g + i;
        const int sx = win_start(min(qxi, p.X - 1), p.X, kx);
        sc[i] = (yz && qxi < p.X && t.x >= sx && t.x < sx + kx) ? 0.f : -INFINITY;
        const int64_t qr = tok_index(p, t.b, qz, qy, min(qxi, p.X - 1), t.h);
        lse[i] = p.lse[qr];
        dsm[i] = p.dsum[qr];
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], kreg[ks], sc, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(da[ks], vreg[ks], dp, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[hb][i] = exp2f(sc[i] - lse[i]);
        sv[hb][i] = pv[hb][i] * (dp[i] - dsm[i]);
      }
    }
    const bf16x8 pbp = __builtin_bit_cast(
        bf16x8, ((u32x4){pack_bf16x2(pv[0][0], pv[0][1]), pack_bf16x2(pv[0][2], pv[0][3]),
                         pack_bf16x2(pv[1][0], pv[1][1]), pack_bf16x2(pv[1][2], pv[1][3])}));
    const bf16x8 pbs = __builtin_bit_cast(
        bf16x8, ((u32x4){pack_bf16x2(sv[0][0], sv[0][1]), pack_bf16x2(sv[0][2], sv[0][3]),
                         pack_bf16x2(sv[1][0], sv[1][1]), pack_bf16x2(sv[1][2], sv[1][3])}));
    wait_lds();  // this wave's Q / dO rows are in LDS
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const bf16x4 q0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, wl + toff[db]));
      const bf16x4 q1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, wl + RBW + toff[db]));
      const bf16x4 o0 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, wl + 2 * RBW + toff[db]));
      const bf16x4 o1 = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, wl + 3 * RBW + toff[db]));
      dk[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_shufflevector(q0, q1, 0, 1, 2, 3, 4, 5, 6, 7), pbs,
                                                       dk[db], 0, 0, 0);
      dv[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_shufflevector(o0, o1, 0, 1, 2, 3, 4, 5, 6, 7), pbp,
                                                       dv[db], 0, 0, 0);
    }
    wait_lds();  // the transposed reads are done before the next pair overwrites the rows
  }
  if (t.valid) {
    constexpr float LN2 = 0.6931471805599453f;  // Q was staged as scale * log2(e) * q
    char* kp = (char*)p.dk + 2 * (kj * D) + 8 * g;
    char* vp = (char*)p.dv + 2 * (kj * D) + 8 * g;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      *(u32x2*)(kp + 32 * db) = (u32x2){pack_bf16x2(dk[db][0] * LN2, dk[db][1] * LN2),
                                        pack_bf16x2(dk[db][2] * LN2, dk[db][3] * LN2)};
      *(u32x2*)(vp + 32 * db) = (u32x2){pack_bf16x2(dv[db][0], dv[db][1]), pack_bf16x2(dv[db][2], dv[db][3])};
    }
  }
#endif
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
static bool mfma_ok(const Na3dBwdParams& p) {
  return p.dil[0] == 1 && p.dil[1] == 1 && p.dil[2] == 1 && p.ker[2] <= 13 && !std::getenv("STRATA_HIP_NA3D_BWD_VALU");
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
  if (sizeof(T) == 2 && D == 64 && mfma_ok(p))
    hipLaunchKernelGGL(na3d_bwd_dq_mfma_kernel, grid, block, 0, st, p);
  else
    hipLaunchKernelGGL((na3d_bwd_dq_kernel<T, D>), grid, block, 0, st, p);
  if (sizeof(T) == 2 && D == 64 && mfma_ok(p))
    hipLaunchKernelGGL(na3d_bwd_dkv_mfma_kernel, grid, block, 0, st, p);
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
    if (k <= 0 || (k % 2) == 0)
      return fail(STRATA_HIP_EINVAL, std::string("na3d_bwd: kernel size must be odd and positive on axis ") + axis[i]);
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
  hipStream_t st = (hipStream_t)stream;
  return a->dtype == STRATA_HIP_BF16 ? launch_bwd_t<bf16>(p, a->head_dim, st) : launch_bwd_t<float>(p, a->head_dim, st);
}
