// NA3D forward for gfx950.
//
// Semantics follow NATTEN's na3d (0.21.5): clamped windows, optional dilation,
// non-causal, softmax over kz*ky*kx keys scaled by `scale`.  Two kernels:
//
//  * na3d_scalar_kernel: one thread per (batch, query, head), fp32 math, used
//    for fp32 inputs and for shapes the MFMA kernel does not cover.
//  * na3d_mfma_kernel:   bf16 inputs, fp32 accumulation.  A workgroup owns a
//    (1, TY, NWX*TX) box of queries of one (batch, head, dilation residue);
//    each wave owns a (TY, TX) = 16-query tile.  The workgroup streams the
//    union of its queries' windows through LDS one pair of key rows (two
//    (z, y) rows of 16+ keys along x) at a time, double buffered.  Per pair a
//    wave computes S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (keys on M,
//    queries on N), applies the window mask and an online softmax, and
//    accumulates O^T += V^T P^T with V^T read from LDS by ds_read_b64_tr_b16.
#include "common.h"

namespace strata {

struct Na3dParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int B, H, D;
  int L[3];
  int org[3];
  int ext[3];
  int ker[3];
  int dil[3];
  float scale;
  int64_t qs[5], ks[5], vs[5], os[5];
};

// ---------------------------------------------------------------------------
// Scalar kernel
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float ld_elem(const T* p) {
  return (float)(*p);
}

template <typename T, int D>
__global__ __launch_bounds__(256) void na3d_scalar_kernel(Na3dParams p, int64_t total) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int h = (int)(idx % p.H);
  int64_t r = idx / p.H;
  const int ex = (int)(r % p.ext[2]);
  r /= p.ext[2];
  const int ey = (int)(r % p.ext[1]);
  r /= p.ext[1];
  const int ez = (int)(r % p.ext[0]);
  const int b = (int)(r / p.ext[0]);

  const int qc[3] = {p.org[0] + ez, p.org[1] + ey, p.org[2] + ex};
  int base[3];
#pragma unroll
  for (int a = 0; a < 3; ++a) {
    const int d = p.dil[a];
    const int g = qc[a] % d;
    const int Lg = sub_len(p.L[a], g, d);
    base[a] = g + d * win_start(qc[a] / d, Lg, p.ker[a]);
  }

  const T* qp = (const T*)p.q + b * p.qs[0] + qc[0] * p.qs[1] + qc[1] * p.qs[2] + qc[2] * p.qs[3] + h * p.qs[4];
  float qv[D];
#pragma unroll
  for (int d = 0; d < D; ++d) qv[d] = ld_elem(qp + d) * p.scale;

  float acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) acc[d] = 0.f;
  float m = -INFINITY, l = 0.f;

  const T* kb = (const T*)p.k + b * p.ks[0] + h * p.ks[4];
  const T* vb = (const T*)p.v + b * p.vs[0] + h * p.vs[4];
  for (int jz = 0; jz < p.ker[0]; ++jz) {
    const int z = base[0] + jz * p.dil[0];
    for (int jy = 0; jy < p.ker[1]; ++jy) {
      const int y = base[1] + jy * p.dil[1];
      for (int jx = 0; jx < p.ker[2]; ++jx) {
        const int x = base[2] + jx * p.dil[2];
        const T* kp = kb + z * p.ks[1] + y * p.ks[2] + x * p.ks[3];
        float s = 0.f;
#pragma unroll
        for (int d = 0; d < D; ++d) s = fmaf(qv[d], ld_elem(kp + d), s);
        const float mn = fmaxf(m, s);
        const float alpha = expf(m - mn);
        const float e = expf(s - mn);
        l = l * alpha + e;
        const T* vp = vb + z * p.vs[1] + y * p.vs[2] + x * p.vs[3];
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] = fmaf(acc[d], alpha, e * ld_elem(vp + d));
        m = mn;
      }
    }
  }
  const float inv = 1.f / l;
  T* op = (T*)p.o + b * p.os[0] + ez * p.os[1] + ey * p.os[2] + ex * p.os[3] + h * p.os[4];
#pragma unroll
  for (int d = 0; d < D; ++d) op[d] = (T)(acc[d] * inv);
}

// ---------------------------------------------------------------------------
// MFMA kernel
// ---------------------------------------------------------------------------
// Tile bookkeeping shared by host and device.
struct Na3dTiles {
  int nxt, nyt, nzt;  // tiles per axis (max over residue classes)
  int nres;           // dil_z * dil_y * dil_x
  int total;          // total workgroups
};

// Swizzle of the 16-byte chunks of one key row in LDS.  f(key) permutes
// 0..7 so that (a) any 8 consecutive keys read at one chunk hit 8 distinct
// chunk slots (K reads, ds_read_b128) and (b) any 4 consecutive keys read at
// a chunk pair {2c, 2c+1} hit 4 distinct pairs (V transpose reads).
__device__ __forceinline__ int swz(int chunk, int key, int cmask) {
  const int f = 2 * (key & 3) + ((key >> 2) & 1);
  return chunk ^ (f & cmask);
}

__device__ __forceinline__ float xor16_max(float x) {
  return fmaxf(x, __shfl_xor(x, 16));
}
__device__ __forceinline__ float xor32_max(float x) {
  return fmaxf(x, __shfl_xor(x, 32));
}

template <int D, int TX, int NWX>
__global__ __launch_bounds__(64 * NWX) void na3d_mfma_kernel(Na3dParams p, Na3dTiles tg) {
  constexpr int TY = 16 / TX;
  constexpr int WQX = NWX * TX;          // workgroup query width along x
  constexpr int LW = (NWX - 1) * TX + 16; // keys per LDS row
  constexpr int CPK = D / 8;              // 16-byte chunks per key
  constexpr int KS = D / 32;              // k-steps of the QK MFMA
  constexpr int DB = D / 16;              // d-blocks of the PV MFMA
  constexpr int ROW = LW * D;             // elements per LDS key row
  constexpr int TENSOR = 2 * ROW;         // two rows per stage
  constexpr int STAGE = 2 * TENSOR;       // K and V
  constexpr int NCHUNK = STAGE / 8;
  constexpr int NT = 64 * NWX;
  constexpr int CPT = (NCHUNK + NT - 1) / NT;  // chunks per thread per stage
  constexpr int CMASK = CPK >= 8 ? 7 : CPK - 1;

  __shared__ __attribute__((aligned(16))) bf16 lds[2 * STAGE];

  // ---- XCD-aware workgroup order: consecutive tiles stay on one XCD ----
  int wg;
  {
    const int id = blockIdx.x, n = gridDim.x;
    const int xcd = id & 7, local = id >> 3;
    const int q = n >> 3, rem = n & 7;
    wg = xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
  }
  const int xt = wg % tg.nxt;
  int t = wg / tg.nxt;
  const int yt = t % tg.nyt;
  t /= tg.nyt;
  const int zt = t % tg.nzt;
  t /= tg.nzt;
  const int res = t % tg.nres;
  t /= tg.nres;
  const int h = t % p.H;
  const int b = t / p.H;

  const int gx = res % p.dil[2];
  const int gy = (res / p.dil[2]) % p.dil[1];
  const int gz = res / (p.dil[2] * p.dil[1]);

  // Sub-grid (one residue class) lengths and query ranges.
  const int Lz = sub_len(p.L[0], gz, p.dil[0]);
  const int Ly = sub_len(p.L[1], gy, p.dil[1]);
  const int Lx = sub_len(p.L[2], gx, p.dil[2]);
  const int qz0 = sub_first(p.org[0], gz, p.dil[0]), qz1 = sub_end(p.org[0], p.ext[0], gz, p.dil[0]);
  const int qy0 = sub_first(p.org[1], gy, p.dil[1]), qy1 = sub_end(p.org[1], p.ext[1], gy, p.dil[1]);
  const int qx0 = sub_first(p.org[2], gx, p.dil[2]), qx1 = sub_end(p.org[2], p.ext[2], gx, p.dil[2]);

  const int iz = qz0 + zt;
  const int y0 = qy0 + yt * TY;
  const int x0 = qx0 + xt * WQX;
  if (iz >= qz1 || y0 >= qy1 || x0 >= qx1) return;  // uniform over the workgroup

  const int kz = p.ker[0], ky = p.ker[1], kx = p.ker[2];
  const int sz = win_start(iz, Lz, kz);
  const int ylast = min(y0 + TY - 1, qy1 - 1);
  const int Y0 = win_start(y0, Ly, ky);
  const int NR = win_start(ylast, Ly, ky) + ky - Y0;  // rows of the y-union
  const int NP = (NR + 1) >> 1;                      // row pairs per z-slice
  const int X0 = win_start(x0, Lx, kx);
  const int nstage = kz * NP;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n16 = lane & 15;
  const int g = lane >> 4;

  // ---- this lane's query ----
  const int xw0 = x0 + wave * TX;
  const int off_w = win_start(min(xw0, qx1 - 1), Lx, kx) - X0;  // wave's key block inside the LDS row
  const int qy = y0 + n16 / TX;
  const int qx = xw0 + n16 % TX;
  const bool qvalid = qy < qy1 && qx < qx1;
  const int qyc = min(qy, qy1 - 1);
  const int qxc = min(qx, qx1 - 1);
  const int sy = win_start(qyc, Ly, ky);
  const int sx = win_start(qxc, Lx, kx);
  uint32_t xbits = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int kxs = X0 + off_w + 4 * g + i;
    xbits |= (kxs >= sx && kxs < sx + kx) ? (1u << i) : 0u;
  }

  const int rz = gz + p.dil[0] * iz;
  bf16x8 qreg[KS];
  {
    const bf16* qp = (const bf16*)p.q + (int64_t)b * p.qs[0] + (int64_t)rz * p.qs[1] +
                     (int64_t)(gy + p.dil[1] * qyc) * p.qs[2] + (int64_t)(gx + p.dil[2] * qxc) * p.qs[3] +
                     (int64_t)h * p.qs[4];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qreg[ks] = *(const bf16x8*)(qp + 32 * ks + 8 * g);
  }

  const bf16* kbase = (const bf16*)p.k + (int64_t)b * p.ks[0] + (int64_t)h * p.ks[4];
  const bf16* vbase = (const bf16*)p.v + (int64_t)b * p.vs[0] + (int64_t)h * p.vs[4];

  // ---- stage loader: global -> registers -> LDS ----
  u32x4 stage_regs[CPT];
  auto load_stage = [&](int s) {
    const int dzi = s / NP;
    const int pr = s - dzi * NP;
    const int zk = sz + dzi;
    const int rzk = gz + p.dil[0] * zk;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ci = tid + c * NT;
      u32x4 val = {0u, 0u, 0u, 0u};
      if (ci < NCHUNK) {
        const int chunk = ci % CPK;
        int tt = ci / CPK;
        const int key = tt % LW;
        tt /= LW;
        const int row = tt & 1;
        const int tensor = tt >> 1;
        const int yr = 2 * pr + row;
        const int xs = X0 + key;
        if (yr < NR && xs < Lx) {
          const int ry = gy + p.dil[1] * (Y0 + yr);
          const int rx = gx + p.dil[2] * xs;
          const int64_t* st = tensor ? p.vs : p.ks;
          const bf16* src = (tensor ? vbase : kbase) + (int64_t)rzk * st[1] + (int64_t)ry * st[2] +
                            (int64_t)rx * st[3] + 8 * chunk;
          val = *(const u32x4*)src;
        }
      }
      stage_regs[c] = val;
    }
  };
  auto store_stage = [&](int buf) {
    bf16* dst = lds + buf * STAGE;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ci = tid + c * NT;
      if (ci < NCHUNK) {
        const int chunk = ci % CPK;
        const int kr = ci / CPK;  // (tensor, row, key) flattened
        const int key = kr % LW;
        *(u32x4*)(dst + kr * D + 8 * swz(chunk, key, CMASK)) = stage_regs[c];
      }
    }
  };

  const float c2 = p.scale * 1.4426950408889634f;  // scores in log2 units
  f32x4 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float mrun = -INFINITY, lrun = 0.f;

  load_stage(0);
  store_stage(0);
  for (int s = 0; s < nstage; ++s) {
    __syncthreads();
    if (s + 1 < nstage) load_stage(s + 1);

    const int buf = s & 1;
    const bf16* Kb = lds + buf * STAGE;
    const bf16* Vb = Kb + TENSOR;
    const int pr = s % NP;

    // S^T = K Q^T for the two rows of the pair.
    f32x4 sacc[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      sacc[r] = (f32x4){0.f, 0.f, 0.f, 0.f};
      const int key = off_w + n16;
      const bf16* krow = Kb + (r * LW + key) * D;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 a = *(const bf16x8*)(krow + 8 * swz(4 * ks + g, key, CMASK));
        sacc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[ks], sacc[r], 0, 0, 0);
      }
    }

    // Window mask + online softmax (4 lanes of a column share one query).
    float tv[8];
    float mloc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int yk = Y0 + 2 * pr + r;
      const bool yok = yk >= sy && yk < sy + ky;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = yok && ((xbits >> i) & 1u);
        const float v = ok ? sacc[r][i] * c2 : -INFINITY;
        tv[4 * r + i] = v;
        mloc = fmaxf(mloc, v);
      }
    }
    mloc = xor16_max(mloc);
    mloc = xor32_max(mloc);
    const float mnew = fmaxf(mrun, mloc);
    const float muse = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = __builtin_amdgcn_exp2f(mrun - muse);
    lrun *= alpha;
#pragma unroll
    for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
    float pv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pv[j] = __builtin_amdgcn_exp2f(tv[j] - muse);
      lrun += pv[j];
    }
    mrun = mnew;
    const u32x4 pw = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]), pack_bf16x2(pv[4], pv[5]),
                      pack_bf16x2(pv[6], pv[7])};
    const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);

    // O^T += V^T P^T.  Lane m of group g reads 4 d-values of key (4g + m/4)
    // of each row; the transpose read hands lane m the 4 keys at d = m.
    {
      const int keyv = off_w + 4 * g + (n16 >> 2);
      const int dq = n16 & 3;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int chunk = 2 * db + (dq >> 1);
        const int eoff = 8 * swz(chunk, keyv, CMASK) + 4 * (dq & 1);
        const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, Vb + keyv * D + eoff));
        const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(LDS_PTR(bf16x4, Vb + (LW + keyv) * D + eoff));
        const bf16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, oacc[db], 0, 0, 0);
      }
    }

    if (s + 1 < nstage) store_stage(buf ^ 1);
  }

  // ---- normalise and store ----
  float ltot = lrun + __shfl_xor(lrun, 16);
  ltot += __shfl_xor(ltot, 32);
  const float inv = 1.f / ltot;
  if (qvalid) {
    const int oz = rz - p.org[0];
    const int oy = gy + p.dil[1] * qy - p.org[1];
    const int ox = gx + p.dil[2] * qx - p.org[2];
    bf16* op = (bf16*)p.o + (int64_t)b * p.os[0] + (int64_t)oz * p.os[1] + (int64_t)oy * p.os[2] +
               (int64_t)ox * p.os[3] + (int64_t)h * p.os[4];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const u32x2 w = {pack_bf16x2(oacc[db][0] * inv, oacc[db][1] * inv),
                       pack_bf16x2(oacc[db][2] * inv, oacc[db][3] * inv)};
      *(u32x2*)(op + 16 * db + 4 * g) = w;
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
template <typename T>
static int launch_scalar(const Na3dParams& p, hipStream_t st) {
  const int64_t total = (int64_t)p.B * p.H * p.ext[0] * p.ext[1] * p.ext[2];
  if (total == 0) return STRATA_HIP_OK;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  switch (p.D) {
#define STRATA_NA3D_SCALAR_CASE(DD)                                                            \
  case DD:                                                                                     \
    hipLaunchKernelGGL((na3d_scalar_kernel<T, DD>), dim3((unsigned)blocks), dim3(threads), 0, st, p, total); \
    break;
    STRATA_NA3D_SCALAR_CASE(8)
    STRATA_NA3D_SCALAR_CASE(16)
    STRATA_NA3D_SCALAR_CASE(32)
    STRATA_NA3D_SCALAR_CASE(64)
    STRATA_NA3D_SCALAR_CASE(128)
#undef STRATA_NA3D_SCALAR_CASE
    default:
      return fail(STRATA_HIP_EUNSUPPORTED, "na3d: head_dim must be one of 8, 16, 32, 64, 128");
  }
  return check_launch("na3d_scalar_kernel");
}

template <int D, int TX, int NWX>
static int launch_mfma_cfg(const Na3dParams& p, hipStream_t st) {
  Na3dTiles tg;
  int nq[3] = {0, 0, 0};
  for (int a = 0; a < 3; ++a)
    for (int g = 0; g < p.dil[a]; ++g) {
      const int n = sub_end(p.org[a], p.ext[a], g, p.dil[a]) - sub_first(p.org[a], g, p.dil[a]);
      nq[a] = n > nq[a] ? n : nq[a];
    }
  constexpr int TY = 16 / TX;
  tg.nzt = nq[0];
  tg.nyt = (nq[1] + TY - 1) / TY;
  tg.nxt = (nq[2] + NWX * TX - 1) / (NWX * TX);
  tg.nres = p.dil[0] * p.dil[1] * p.dil[2];
  const int64_t total = (int64_t)tg.nxt * tg.nyt * tg.nzt * tg.nres * p.H * p.B;
  if (total == 0) return STRATA_HIP_OK;
  if (total > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "na3d: problem too large for one launch");
  tg.total = (int)total;
  hipLaunchKernelGGL((na3d_mfma_kernel<D, TX, NWX>), dim3(tg.total), dim3(64 * NWX), 0, st, p, tg);
  return check_launch("na3d_mfma_kernel");
}

template <int D>
static int launch_mfma_d(const Na3dParams& p, hipStream_t st) {
  const int kx = p.ker[2];
  if (kx == 1) return launch_mfma_cfg<D, 16, 4>(p, st);
  if (kx <= 9) return launch_mfma_cfg<D, 8, 4>(p, st);
  if (kx <= 13) return launch_mfma_cfg<D, 4, 4>(p, st);
  return launch_mfma_cfg<D, 2, 4>(p, st);  // kx <= 15
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace strata

using namespace strata;

extern "C" int strata_hip_na3d_fwd(const strata_hip_na3d_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "na3d: null args");
  if (!a->q || !a->k || !a->v || !a->out) return fail(STRATA_HIP_EINVAL, "na3d: null tensor pointer");
  if (a->dtype != STRATA_HIP_F32 && a->dtype != STRATA_HIP_BF16)
    return fail(STRATA_HIP_EINVAL, "na3d: dtype must be f32 or bf16");
  if (a->batch < 0 || a->heads <= 0 || a->head_dim <= 0) return fail(STRATA_HIP_EINVAL, "na3d: bad batch/heads/head_dim");
  static const char* axis = "zyx";
  for (int i = 0; i < 3; ++i) {
    const int L = a->grid[i], k = a->kernel[i], d = a->dilation[i];
    if (L <= 0) return fail(STRATA_HIP_EINVAL, std::string("na3d: grid size must be positive on axis ") + axis[i]);
    if (k <= 0 || (k % 2) == 0)
      return fail(STRATA_HIP_EINVAL, std::string("na3d: kernel size must be odd and positive on axis ") + axis[i]);
    if (d <= 0) return fail(STRATA_HIP_EINVAL, std::string("na3d: dilation must be positive on axis ") + axis[i]);
    if ((int64_t)k * d > L)
      return fail(STRATA_HIP_EINVAL,
                  std::string("na3d: kernel_size * dilation exceeds the token grid on axis ") + axis[i]);
    if (a->q_origin[i] < 0 || a->q_extent[i] < 0 || a->q_origin[i] + a->q_extent[i] > L)
      return fail(STRATA_HIP_EINVAL, std::string("na3d: query box outside the grid on axis ") + axis[i]);
  }
  Na3dParams p;
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.o = a->out;
  p.B = a->batch;
  p.H = a->heads;
  p.D = a->head_dim;
  for (int i = 0; i < 3; ++i) {
    p.L[i] = a->grid[i];
    p.org[i] = a->q_origin[i];
    p.ext[i] = a->q_extent[i];
    p.ker[i] = a->kernel[i];
    p.dil[i] = a->dilation[i];
  }
  for (int i = 0; i < 5; ++i) {
    p.qs[i] = a->q_stride[i];
    p.ks[i] = a->k_stride[i];
    p.vs[i] = a->v_stride[i];
    p.os[i] = a->o_stride[i];
  }
  p.scale = a->scale;
  if ((int64_t)p.B * p.ext[0] * p.ext[1] * p.ext[2] == 0) return STRATA_HIP_OK;
  hipStream_t st = (hipStream_t)stream;

  if (a->dtype == STRATA_HIP_F32) return launch_scalar<float>(p, st);

  bool mfma_ok = (p.D == 32 || p.D == 64 || p.D == 128) && p.ker[2] <= 15;
  if (mfma_ok) {
    const void* ptrs[4] = {p.q, p.k, p.v, p.o};
    const int64_t* strides[4] = {p.qs, p.ks, p.vs, p.os};
    for (int t = 0; t < 4; ++t) {
      if (!aligned16(ptrs[t])) mfma_ok = false;
      for (int i = 0; i < 5; ++i)
        if (strides[t][i] % 8 != 0) mfma_ok = false;
    }
  }
  if (!mfma_ok) return launch_scalar<bf16>(p, st);
  switch (p.D) {
    case 32:
      return launch_mfma_d<32>(p, st);
    case 64:
      return launch_mfma_d<64>(p, st);
    default:
      return launch_mfma_d<128>(p, st);
  }
}
