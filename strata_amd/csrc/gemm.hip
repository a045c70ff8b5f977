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
// Two kernels: gemm_dma_kernel (256 x 256 tiles, 8 waves, global->LDS
// streaming; the last K step masked when K is not a multiple of 64) for every
// GEMM of the block and the rollout, plain or with a fused epilogue, and
// gemm_bias_act_kernel (128 x 128 tiles, register-staged loads) for row
// strides too long for the former's 32-bit lane offsets.
#include "gemm.h"

namespace strata {

__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3) equals
  // x * sigmoid(2u) = x / (1 + 2^(-2u log2(e))): one exp2 and one reciprocal.
  constexpr float k1 = 2.f * 1.4426950408889634f * 0.7978845608028654f;
  const float t = x * fmaf(k1 * 0.044715f, x * x, k1);
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-t));
}
// d/dx gelu_tanh(x) = s + 2 x s (1 - s) u'(x) with s = sigmoid(2u) as above and
// u' = sqrt(2/pi) (1 + 3 * 0.044715 x^2) (the backward of the MLP's GELU).
__device__ __forceinline__ float gelu_tanh_grad(float x) {
  constexpr float c = 0.7978845608028654f;
  constexpr float k1 = 2.f * 1.4426950408889634f * c;
  const float t = x * fmaf(k1 * 0.044715f, x * x, k1);
  const float s = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-t));
  const float du2 = 2.f * c * fmaf(3.f * 0.044715f, x * x, 1.f);
  return fmaf(x * s * (1.f - s), du2, s);
}
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.7071067811865476f)); }
// sigmoid(x) = 1 / (1 + 2^(-x log2 e)); saturates to 0 / 1 through inf / 0.
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}
// sigmoid'(x) = s (1 - s): the gate's backward.
__device__ __forceinline__ float sigmoid_grad(float x) {
  const float s = sigmoid_fast(x);
  return s * (1.f - s);
}
__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == STRATA_HIP_ACT_GELU_TANH) return gelu_tanh(v);
  if (act == STRATA_HIP_ACT_GELU_ERF) return gelu_erf(v);
  if (act == STRATA_HIP_ACT_SIGMOID) return sigmoid_fast(v);
  if (act == STRATA_HIP_ACT_GELU_TANH_GRAD) return gelu_tanh_grad(v);
  if (act == STRATA_HIP_ACT_SIGMOID_GRAD) return sigmoid_grad(v);
  return v;
}
__device__ __forceinline__ float combine(float o, float r, int res_op) {
  return res_op == STRATA_HIP_RES_MUL ? o * r : o + r;
}
// Compile-time forms for the large-tile kernel: one instance per activation
// and residual mode keeps its epilogue straight-line (a runtime activation
// code makes every element branch over all four activations).
enum { RES_NONE_T = 0, RES_ADD_T = 1, RES_MUL_T = 2 };
template <int ACT>
__device__ __forceinline__ float act_t(float v) {
  if constexpr (ACT == STRATA_HIP_ACT_GELU_TANH) return gelu_tanh(v);
  else if constexpr (ACT == STRATA_HIP_ACT_GELU_ERF) return gelu_erf(v);
  else if constexpr (ACT == STRATA_HIP_ACT_SIGMOID) return sigmoid_fast(v);
  else if constexpr (ACT == STRATA_HIP_ACT_GELU_TANH_GRAD) return gelu_tanh_grad(v);
  else if constexpr (ACT == STRATA_HIP_ACT_SIGMOID_GRAD) return sigmoid_grad(v);
  else return v;
}
template <int RES>
__device__ __forceinline__ float combine_t(float o, float r) {
  return RES == RES_MUL_T ? o * r : o + r;
}

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
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = apply_act(v[e], p.act);
        if (full) {
          if (p.res) {
            const u32x2 rw = *(const u32x2*)(p.res + gm * p.ldr + gn);
            v[0] = combine(v[0], bf16_lo(rw[0]), p.res_op);
            v[1] = combine(v[1], bf16_hi(rw[0]), p.res_op);
            v[2] = combine(v[2], bf16_lo(rw[1]), p.res_op);
            v[3] = combine(v[3], bf16_hi(rw[1]), p.res_op);
          }
          const u32x2 ow = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
          *(u32x2*)(p.out + gm * p.ldo + gn) = ow;
        } else {
          for (int e = 0; e < 4 && gn + e < p.N; ++e) {
            float o = v[e];
            if (p.res) o = combine(o, (float)p.res[gm * p.ldr + gn + e], p.res_op);
            p.out[gm * p.ldo + gn + e] = (bf16)o;
          }
        }
      }
    }
  }
}

// Epilogue for 4 consecutive output columns gn..gn+3 of row gm.
__device__ __forceinline__ void store_quad(const GemmParams& p, int64_t gm, int64_t gn, float v0, float v1, float v2,
                                           float v3) {
  float v[4] = {v0, v1, v2, v3};
  if (gm >= p.M || gn >= p.N) return;
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
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = apply_act(v[e], p.act);
  if (full) {
    if (p.res) {
      const u32x2 rw = *(const u32x2*)(p.res + gm * p.ldr + gn);
      v[0] = combine(v[0], bf16_lo(rw[0]), p.res_op);
      v[1] = combine(v[1], bf16_hi(rw[0]), p.res_op);
      v[2] = combine(v[2], bf16_lo(rw[1]), p.res_op);
      v[3] = combine(v[3], bf16_hi(rw[1]), p.res_op);
    }
    const u32x2 ow = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    *(u32x2*)(p.out + gm * p.ldo + gn) = ow;
  } else {
    for (int e = 0; e < 4 && gn + e < p.N; ++e) {
      float o = v[e];
      if (p.res) o = combine(o, (float)p.res[gm * p.ldr + gn + e], p.res_op);
      p.out[gm * p.ldo + gn + e] = (bf16)o;
    }
  }
}

// Swizzle of the 16-byte chunks of an LDS row (CH chunks of a BK-wide row):
// the 16 consecutive rows that one pass of a ds_read_b128 serves, all at the
// same logical chunk, land on 16 distinct 16-byte bank groups.
//   CH = 8 (128-byte rows): two rows share a 256-byte bank line;
//   CH = 4 (64-byte rows): four rows share one.
template <int CH>
__device__ __forceinline__ int gswz(int chunk, int row) {
  if constexpr (CH == 8) return chunk ^ ((row & 7) ^ ((row >> 3) & 1));
  else return chunk ^ ((row >> 2) & 3);
}

// Large-tile GEMM (K a multiple of 8): a BM x BN output tile per workgroup of
// WGM x WGN waves (128 x 64 each, v_mfma_f32_32x32x16_bf16).  A/B tiles of BK
// columns stream from global memory straight into a double-buffered LDS ring
// (buffer_load ... lds) one stage ahead of the MFMAs, one barrier per stage.
// The ring runs on across the tiles of the persistent walk: the last K step
// of a tile issues the next tile's first stage, whose copy then lands while
// the epilogue runs in the other slot.
// SAVE: also write act'(pre-activation) (GELU(tanh) only) to p.out2, for a
// backward that then needs no recomputed GEMM.
template <int BM, int BN, int WGM, int WGN, int BK, int NST, int ACT, int RES, bool SAVE = false,
          bool KTAIL = false>
__device__ __forceinline__ void gemm_dma_body(const GemmParams& p) {
  constexpr int NW = WGM * WGN;
  constexpr int WTM = BM / WGM;  // 128
  constexpr int WTN = BN / WGN;  // 64
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int ROWB = BK * 2;            // bytes of one tile row in a stage
  constexpr int CH = ROWB / 16;           // 16-byte chunks per row
  constexpr int RPC = 1024 / ROWB;        // rows per 1-KiB DMA
  constexpr int XB = BM * ROWB;           // bytes of the x tile
  constexpr int XCH = XB / 1024;          // 1-KiB DMAs of the x tile
  constexpr int STAGE = XB + BN * ROWB;
  constexpr int LPW = STAGE / 1024 / NW;  // 1-KiB DMAs per wave per stage
  constexpr int HM = FM / 2;              // accumulator rows (of 32) per epilogue half
  constexpr int SLAB = HM * 32 * WTN * 2;  // one wave's epilogue slab: half its tile
  static_assert(CH == 4 || CH == 8, "BK must be 32 or 64");
  static_assert(NST == 2, "double-buffered ring");
  static_assert(WTM == 128 && WTN == 64 && STAGE % (1024 * NW) == 0, "wave tile / stage layout");
  static_assert(NW * SLAB <= STAGE, "the epilogue slabs fit one ring slot");
  __shared__ __attribute__((aligned(1024))) char lds[NST * STAGE];  // ring; slabs in the slot last read

  const int tid = (int)__builtin_amdgcn_workitem_id_x();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int wm = wave / WGN, wn = wave % WGN;
  const int l32 = lane & 31, hi = lane >> 5;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

  // Persistent: a workgroup walks tiles id, id + grid, ...  With a grid that
  // is a multiple of 8, tile index t stays on the XCD that runs workgroup id
  // (the dispatcher deals workgroups round-robin over the 8 XCDs), and each
  // XCD takes a contiguous block of tiles, 32 neighbours in flight at once.
  // Tiles in groups of GRP row panels x every column panel, row panel fastest:
  // an XCD's 32 concurrent tiles share 4 panels of x and 8 of w (measured at
  // the block's shapes with the stores below: 1-2% faster than one row panel
  // x all columns).
  const int ntiles = p.mt * p.nt;
  const int wg_id = (int)__builtin_amdgcn_workgroup_id_x();
  auto tile_origin = [&](int t, int64_t& m0, int64_t& n0) {
    const int xcd = t & 7, local = t >> 3, q = ntiles >> 3, rem = ntiles & 7;
    const int wg = xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
    constexpr int GRP = 4;
    const int gi = wg / (GRP * p.nt), li = wg % (GRP * p.nt);
    const int gmn = min(GRP, p.mt - gi * GRP);  // row panels in this (possibly last) group
    m0 = (int64_t)(gi * GRP + li % gmn) * BM;
    n0 = (int64_t)(li / gmn) * BN;
  };

  // DMA j = c / NW of a stage (c = j*NW + wave) covers RPC rows of the x tile
  // (c < XCH) or of the w tile; lane i fills row RPC*(c%XCH) + i/CH, slot i%CH.
  // Rows past M (or N) get the out-of-range offset and read as zero.
  auto dma_off = [&](int j, int64_t m0, int64_t n0) -> uint32_t {
    const int c = j * NW + wave;
    const bool isw = c >= XCH;
    const int row = RPC * (isw ? c - XCH : c) + lane / CH;
    const int lc = gswz<CH>(lane % CH, row);
    const bool ok = (isw ? n0 : m0) + row < (isw ? p.N : p.M);
    return ok ? (uint32_t)(row * (isw ? p.ldw : p.ldx) * 2 + lc * 16) : OOB;
  };
  // KTAIL (K % BK != 0; separate instances, so that the others keep their
  // registers): the last stage holds KT = K % BK columns (a multiple of 8); a
  // lane's chunk of copy j past them takes the out-of-range offset and reads
  // as zero (beyond K lies the row's padding or, on the last row, past the
  // end of the tensor).  The chunk depends on the lane and the row inside the
  // tile only; it is recomputed at that stage from an opaque copy of the lane
  // id (a mask held across the tile walk costs more registers).
  const int nk = (int)(KTAIL ? (p.K + BK - 1) / BK : p.K / BK);
  // The copies of stage kt into slot buf; PART: both tiles (ALL), or only the
  // x tile's (XS) or the w tile's (WS) copies.  Copy j reads w exactly when
  // j * NW >= XCH (XCH is a multiple of NW), so the split is compile-time.
  enum { ALL = 0, XS = 1, WS = 2 };
  static_assert(XCH % NW == 0, "a copy index reads x or w for every wave");
  auto issue_at = [&](int64_t m0, int64_t n0, const uint32_t* vo, int kt, int buf, auto part) {
    constexpr int PART = decltype(part)::value;
    const u32x4 rx = make_rsrc((const char*)(p.x + m0 * p.ldx) + (int64_t)kt * BK * 2, OOB);
    const u32x4 rw = make_rsrc((const char*)(p.w + n0 * p.ldw) + (int64_t)kt * BK * 2, OOB);
    const uint32_t dst = lds_base + buf * STAGE + wave * 1024;
    auto mine = [](int j) { return PART == ALL || (PART == WS) == (j * NW >= XCH); };
    if (KTAIL && kt == nk - 1) {  // uniform: the ragged last stage
      int ln = lane;
      asm volatile("" : "+v"(ln));
#pragma unroll
      for (int j = 0; j < LPW; ++j) {
        if (!mine(j)) continue;
        const bool isw = j * NW >= XCH;
        const int row = RPC * (isw ? j * NW + wave - XCH : j * NW + wave) + ln / CH;
        const bool ok = gswz<CH>(ln % CH, row) * 8 < (int)(p.K % BK);
        dma_row16(isw ? rw : rx, dst + j * NW * 1024, ok ? vo[j] : OOB);
      }
    } else {
#pragma unroll
      for (int j = 0; j < LPW; ++j)
        if (mine(j)) dma_row16(j * NW >= XCH ? rw : rx, dst + j * NW * 1024, vo[j]);
    }
  };
  // A tile's first stage, with offsets computed on the spot.
  auto issue_first = [&](int64_t m0, int64_t n0, int buf) {
    uint32_t vo[LPW];
#pragma unroll
    for (int j = 0; j < LPW; ++j) vo[j] = dma_off(j, m0, n0);
    issue_at(m0, n0, vo, 0, buf, std::integral_constant<int, ALL>{});
  };

  // LDS read offsets of the MFMA operands for K sub-steps kk = 0, 1; kk = 2, 3
  // (64-wide stages) flip bit 2 of the chunk, i.e. byte offset ^ 64.
  uint32_t aoff[FN][2], boff[FM][2];
#pragma unroll
  for (int i = 0; i < FN; ++i) {
    const int row = wn * WTN + 32 * i + l32;
    for (int kk = 0; kk < 2; ++kk) aoff[i][kk] = XB + row * ROWB + gswz<CH>(2 * kk + hi, row) * 16;
  }
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int row = wm * WTM + 32 * j + l32;
    for (int kk = 0; kk < 2; ++kk) boff[j][kk] = row * ROWB + gswz<CH>(2 * kk + hi, row) * 16;
  }

  // The bias as the first K step's C operand: binit[i][4q + e] holds column
  // 32i + 8q + 4hi + e of the wave tile.  EARLY_BIAS: the next tile's bias is
  // loaded at the start of the epilogue (all eight loads in flight together) and
  // converted at its end, so that the loads' latency hides behind the epilogue.
  // The instances with the saved derivative, GELU(erf), or the GELU derivative
  // beside a residual spill with it: they load at the tile's start.
  constexpr bool EARLY_BIAS = !SAVE && ACT != STRATA_HIP_ACT_GELU_ERF &&
                              !(RES != RES_NONE_T && ACT == STRATA_HIP_ACT_GELU_TANH_GRAD);
  f32x16 binit[FN];
  // bb[i][q]: the bf16 pairs of columns n0x + wn * WTN + 32i + 8q + 4hi + (0..3).
  // Uniform branches; a column panel inside the matrix loads with no per-lane
  // condition (a divergent if / else writing the same registers makes the
  // compiler wait for each load before issuing the next).
  auto load_bias = [&](int64_t n0x, u32x2 (&bb)[FN][4]) {
    const int64_t gb = n0x + wn * WTN + 4 * hi;
    if (!p.bias) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) bb[i][q] = (u32x2){0u, 0u};
    } else if (n0x + BN <= p.N) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) bb[i][q] = *(const u32x2*)(p.bias + gb + 32 * i + 8 * q);
    } else {  // the ragged last column panel
      const uint16_t* b16 = (const uint16_t*)p.bias;
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          u32x2 w2 = {0u, 0u};
          for (int e = 0; e < 4; ++e) {
            const int64_t gn = gb + 32 * i + 8 * q + e;
            if (gn < p.N) w2[e >> 1] |= (uint32_t)b16[gn] << (16 * (e & 1));
          }
          bb[i][q] = w2;
        }
    }
  };
  // bb -> binit.  The empty asm takes the loaded registers as its output, so the
  // compiler waits for the loads here, once, and the walk carries only computed
  // registers (with the loads' registers carried to the next tile, it waited for
  // them, and so for every store issued before, at the head of the next K loop).
  auto settle_bias = [&](u32x2 (&bb)[FN][4]) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        asm volatile("" : "+v"(bb[i][q]));
        binit[i][4 * q + 0] = bf16_lo(bb[i][q][0]);
        binit[i][4 * q + 1] = bf16_hi(bb[i][q][0]);
        binit[i][4 * q + 2] = bf16_lo(bb[i][q][1]);
        binit[i][4 * q + 3] = bf16_hi(bb[i][q][1]);
      }
  };
  if (EARLY_BIAS && wg_id < ntiles) {
    int64_t m0f, n0f;
    tile_origin(wg_id, m0f, n0f);
    u32x2 bb[FN][4];
    load_bias(n0f, bb);
    settle_bias(bb);
  }

  // Ring slots: `rd` holds the next stage to read, `wr` takes the next issue
  // (and, after a tile's last K step, that tile's epilogue slabs).
  int rd = 0, wr = 1;
  bool first_in_flight = false;  // the current tile's first stage was issued by the previous tile
  for (int t = wg_id; t < ntiles; t += (int)gridDim.x) {
  int64_t m0, n0;
  tile_origin(t, m0, n0);
  const int tn = t + (int)gridDim.x;  // the next tile of this workgroup
  int64_t m0n = 0, n0n = 0;
  if (tn < ntiles) tile_origin(tn, m0n, n0n);

  uint32_t voff[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) voff[j] = dma_off(j, m0, n0);
  // Slot rd was last read two K steps ago (or never): no barrier needed.
  if (!first_in_flight) issue_at(m0, n0, voff, 0, rd, std::integral_constant<int, ALL>{});

  // The bias enters as the C operand of each accumulator's first MFMA (no
  // zero fill, no add in the epilogue).
  const int64_t gn0 = n0 + wn * WTN, gm0 = m0 + wm * WTM;
  const bool full = m0 + BM <= p.M && n0 + BN <= p.N;  // uniform
  if constexpr (!EARLY_BIAS) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t gn = gn0 + 32 * i + 8 * q + 4 * hi;
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.bias) {
          if (full || gn + 4 <= p.N) {
            const u32x2 w2 = *(const u32x2*)(p.bias + gn);
            bv[0] = bf16_lo(w2[0]);
            bv[1] = bf16_hi(w2[0]);
            bv[2] = bf16_lo(w2[1]);
            bv[3] = bf16_hi(w2[1]);
          } else {
            for (int e = 0; e < 4; ++e) bv[e] = gn + e < p.N ? (float)p.bias[gn + e] : 0.f;  // ragged last columns
          }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) binit[i][4 * q + e] = bv[e];
      }
  }

  f32x16 acc[FN][FM];
  first_in_flight = false;
  // One K step; FIRST: the step that starts every accumulator from the bias.
  auto kstep = [&](int kt, auto first) {
    constexpr bool FIRST = decltype(first)::value;
    // The wait is for everything issued: the stage read now (issued one step
    // ago) and, at a tile's first step, the previous tile's output stores (the
    // compiler holds the registers of their data until they complete, so a
    // wait that left them in flight would stall on the first LDS reads
    // instead).
    wait_vmcnt(0);
    lds_barrier();  // the stage has landed for every wave; slot wr is free
    // The next stage's copies in two bursts, x here and w after the first
    // sub-step's MFMAs (A/B at the block's shapes, bit-identical: 1.5-5%
    // faster than all eight of a wave's copies here; later in the step,
    // spread further, all after the first sub-step, or the two waves of a
    // SIMD out of step: no faster or slower).  The copies cost the K loop
    // 25-35% with a whole stage in flight and 3-10% with half of one.
    const int wr_now = wr;
    if (kt + 1 < nk) {
      issue_at(m0, n0, voff, kt + 1, wr, std::integral_constant<int, XS>{});
    } else if (tn < ntiles) {
      // The next tile's first stage.  Its origin passes through an empty asm
      // so that its lane offsets are computed here, not hoisted out of the K
      // loop into registers held across it.
      int64_t mn = m0n, nn = n0n;
      asm volatile("" : "+s"(mn), "+s"(nn));
      issue_first(mn, nn, wr);
      first_in_flight = true;
    }
    const char* st = lds + rd * STAGE;
    rd ^= 1;
    wr ^= 1;
    // Operand fragments double-buffered in registers: the LDS reads of K
    // sub-step kk + 1 are issued before the MFMAs of kk, so their latency
    // hides behind those MFMAs.
    bf16x8 af[2][FN], bfr[2][FM];
    auto load_frags = [&](int kk, int buf) {
#pragma unroll
      for (int i = 0; i < FN; ++i) af[buf][i] = *(const bf16x8*)(st + (aoff[i][kk & 1] ^ ((kk >> 1) * 64)));
#pragma unroll
      for (int j = 0; j < FM; ++j) bfr[buf][j] = *(const bf16x8*)(st + (boff[j][kk & 1] ^ ((kk >> 1) * 64)));
    };
    load_frags(0, 0);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int cb = kk & 1;
      if (kk + 1 < BK / 16) load_frags(kk + 1, cb ^ 1);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[cb][i], bfr[cb][j],
                                                             FIRST && kk == 0 ? binit[i] : acc[i][j], 0, 0, 0);
      if (kk == 0 && kt + 1 < nk) {
        __builtin_amdgcn_sched_barrier(0);
        issue_at(m0, n0, voff, kt + 1, wr_now, std::integral_constant<int, WS>{});
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // Let the scheduler interleave the LDS reads of the next sub-step with
    // the MFMAs of the current one (measured 1-3% faster than the default
    // order at the block's shapes; explicit sched_group_barrier groups gave
    // the default order back).
    __builtin_amdgcn_iglp_opt(1);
  };
  kstep(0, std::true_type{});
  for (int kt = 1; kt < nk; ++kt) kstep(kt, std::false_type{});

  // ---- epilogue through LDS, in two halves of the wave tile ----
  // Phase 1: activation on the accumulators (the bias is already in them), bf16 into this wave's
  // slab (64 rows of SRB bytes, 16-byte chunks swizzled by row) in ring slot wr, the slot the
  // last K step read; slot rd meanwhile receives the next tile's first stage.
  // Phase 2: each lane reads 16 contiguous bytes of a row, combines the
  // residual read the same way, and writes 16 bytes: CPR lanes cover a row.
  // A half's slab rows are read back together (its LDS reads in flight at
  // once, one wait) and a tile inside the matrix takes one branch for the
  // whole half (a bounds branch per row made every row wait for its own LDS
  // read before its store).
  // Loads and stores share vmcnt on gfx9 (a load issued after a store waits
  // for it), so every residual load is issued before the first store.  The
  // slab is rewritten by the second half only after the first half's reads
  // (one wave, in order).
  constexpr int SRB = WTN * 2, CPR = WTN / 8, RPI = 64 / CPR, NIT = WTM / RPI, NH = NIT / 2;
  u32x2 nb[FN][4];  // the next tile's bias (after the last tile: column panel 0's, unused)
  if constexpr (EARLY_BIAS) load_bias(n0n, nb);
  lds_barrier();  // every wave is done reading the last stage
  char* slab = lds + wr * STAGE + wave * SLAB;
  const int c = lane % CPR;  // logical 16-byte chunk = 8 output columns
  const int64_t gn = gn0 + 8 * c;
  u32x4 r4[NIT];
  // Phase 1 for one half: f(accumulator) -> bf16 into the slab.
  auto to_slab = [&](int half, auto f) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = 32 * i + 8 * q + 4 * hi;  // local column of this lane's quad
#pragma unroll
        for (int jj = 0; jj < HM; ++jj) {
          const int j = half * HM + jj;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = f(acc[i][j][4 * q + e]);
          const int ml = 32 * jj + l32;
          const u32x2 w2 = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
          *(u32x2*)(slab + ml * SRB + (((nl >> 3) ^ (ml & 7)) << 4) + 8 * hi) = w2;
        }
      }
  };
  // Phase 2 for one half, to dst; WITH_RES: combine the residual (the output
  // pass; the saved derivative takes none).
  // GR rows are read back per group: all of a half, or half of one in the SAVE
  // instance, whose accumulators all stay live through the first half.
  constexpr int GR = SAVE ? NH / 2 : NH;
  auto from_slab = [&](int half, bf16* dst, auto with_res) {
    constexpr bool WR = decltype(with_res)::value && RES != RES_NONE_T;
    const int64_t gmh = gm0 + half * (WTM / 2) + lane / CPR;  // this lane's row for slab row group 0
#pragma unroll
    for (int k0 = 0; k0 < NH; k0 += GR) {
      u32x4 w4[GR];
#pragma unroll
      for (int k = 0; k < GR; ++k) {
        const int sl = RPI * (k0 + k) + lane / CPR;  // row of the slab
        w4[k] = *(const u32x4*)(slab + sl * SRB + ((c ^ (sl & 7)) << 4));
      }
      auto combined = [&](int k) {
        u32x4 o = w4[k];
        if constexpr (WR) {
          const u32x4& r = r4[half * NH + k0 + k];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = pack_bf16x2(combine_t<RES>(bf16_lo(w4[k][e]), bf16_lo(r[e])),
                               combine_t<RES>(bf16_hi(w4[k][e]), bf16_hi(r[e])));
        }
        return o;
      };
      // Streaming stores: the output is not read again here, and a tile-round's
      // outputs (32 MB over the grid) would otherwise push the x and w panels
      // out of L2 (M = 131072, N = 4096, K = 1024 with GELU: 1.32 -> 1.27 ms).
      if (full) {
#pragma unroll
        for (int k = 0; k < GR; ++k)
          __builtin_nontemporal_store(combined(k), (u32x4*)(dst + (gmh + RPI * (k0 + k)) * p.ldo + gn));
      } else {
#pragma unroll
        for (int k = 0; k < GR; ++k) {
          const int64_t gm = gmh + RPI * (k0 + k);
          if (gm < p.M && gn + 8 <= p.N) {
            __builtin_nontemporal_store(combined(k), (u32x4*)(dst + gm * p.ldo + gn));
          } else if (gm < p.M && gn < p.N) {
            for (int e = 0; e < 8 && gn + e < p.N; ++e) {  // ragged last columns
              const uint32_t wd = w4[k][e >> 1];
              float ov = (e & 1) ? bf16_hi(wd) : bf16_lo(wd);
              if constexpr (WR) ov = combine_t<RES>(ov, (float)p.res[gm * p.ldr + gn + e]);
              dst[gm * p.ldo + gn + e] = (bf16)ov;
            }
          }
        }
      }
    }
  };
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    to_slab(half, [](float x) { return act_t<ACT>(x); });
    if constexpr (RES != RES_NONE_T) {
      // All residual rows, into the registers the first half's accumulators
      // freed (loaded before that conversion, even the first half's rows
      // alone spill 4-14 VGPRs).
      if (half == 0) {
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          const int64_t gm = gm0 + RPI * it + lane / CPR;
          r4[it] = (u32x4){0u, 0u, 0u, 0u};
          if (full || (gm < p.M && gn + 8 <= p.N)) r4[it] = *(const u32x4*)(p.res + gm * p.ldr + gn);
        }
      }
    }
    from_slab(half, p.out, std::true_type{});
    if constexpr (SAVE) {  // the derivative of the same half through the same slab, to out2
      static_assert(ACT == STRATA_HIP_ACT_GELU_TANH, "SAVE: GELU(tanh) only");
      // recomputed, not shared with the first pass: sharing would hold the whole
      // half's sigmoids in registers between the two passes
      to_slab(half, [](float xv) {
        asm volatile("" : "+v"(xv));
        return gelu_tanh_grad(xv);
      });
      from_slab(half, p.out2, std::false_type{});
    }
  }
  if constexpr (EARLY_BIAS) settle_bias(nb);
  }  // tiles
}

// One 256 x 256 workgroup of 8 waves per CU, K step 64, double-buffered
// 128 KiB ring.  (Measured alternatives at the block's shapes, all slower:
// 256 x 128 tiles at two workgroups per CU; K step 32 with 3-5 stages; four
// waves of 128 x 128 with the accumulators in AGPRs.)
template <int ACT, int RES, bool SAVE = false, bool KTAIL = false>
__global__ __launch_bounds__(512, 1) void gemm_dma_kernel(GemmParams p) {
  gemm_dma_body<256, 256, 2, 4, 64, 2, ACT, RES, SAVE, KTAIL>(p);
}

template <int ACT>
static void launch_dma_act(const GemmParams& p, dim3 grid, hipStream_t st) {
  auto go = [&](auto ktail) {
    constexpr bool KT = decltype(ktail)::value;
    if (!p.res)
      hipLaunchKernelGGL((gemm_dma_kernel<ACT, RES_NONE_T, false, KT>), grid, dim3(512), 0, st, p);
    else if (p.res_op == STRATA_HIP_RES_MUL)
      hipLaunchKernelGGL((gemm_dma_kernel<ACT, RES_MUL_T, false, KT>), grid, dim3(512), 0, st, p);
    else
      hipLaunchKernelGGL((gemm_dma_kernel<ACT, RES_ADD_T, false, KT>), grid, dim3(512), 0, st, p);
  };
  if (p.K % 64) go(std::true_type{});
  else go(std::false_type{});
}

// Compute units of the current device (cached per device).
static int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
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

namespace strata {

// Argument checks shared by the GEMM entry points; fills p (tile counts aside).
static int gemm_params(const strata_hip_gemm_args* a, GemmParams& p) {
  if (!a) return fail(STRATA_HIP_EINVAL, "gemm: null args");
  if (a->m < 0 || a->n < 0 || a->k <= 0) return fail(STRATA_HIP_EINVAL, "gemm: bad m/n/k");
  if (a->m > 0 && a->n > 0) {
    if (!a->x || !a->w || !a->out) return fail(STRATA_HIP_EINVAL, "gemm: null x, w or out");
    if (a->k % 8 != 0) return fail(STRATA_HIP_EINVAL, "gemm: k must be a multiple of 8");
    if (a->ldx < a->k || a->ldw < a->k || a->ldo < a->n || (a->residual && a->ldr < a->n))
      return fail(STRATA_HIP_EINVAL, "gemm: row stride smaller than the row length");
    // The epilogue stores and the residual loads move 16 bytes of a row at a time.
    if (a->ldx % 8 || a->ldw % 8 || a->ldo % 8 || (a->residual && a->ldr % 8))
      return fail(STRATA_HIP_EINVAL, "gemm: row strides must be multiples of 8 elements");
    if (((uintptr_t)a->x & 15) || ((uintptr_t)a->w & 15) || ((uintptr_t)a->out & 15) ||
        (a->residual && ((uintptr_t)a->residual & 15)) || (a->bias && ((uintptr_t)a->bias & 7)))
      return fail(STRATA_HIP_EINVAL, "gemm: x, w, out and residual must be 16-byte aligned, bias 8-byte aligned");
  }
  if (a->act < STRATA_HIP_ACT_NONE || a->act > STRATA_HIP_ACT_SIGMOID_GRAD) return fail(STRATA_HIP_EINVAL, "gemm: bad act");
  if (a->res_op != STRATA_HIP_RES_ADD && a->res_op != STRATA_HIP_RES_MUL) return fail(STRATA_HIP_EINVAL, "gemm: bad res_op");
  p.x = (const bf16*)a->x;
  p.w = (const bf16*)a->w;
  p.bias = (const bf16*)a->bias;
  p.res = (const bf16*)a->residual;
  p.out = (bf16*)a->out;
  p.out2 = nullptr;
  p.M = a->m;
  p.N = a->n;
  p.K = a->k;
  p.ldx = a->ldx;
  p.ldw = a->ldw;
  p.ldr = a->ldr;
  p.ldo = a->ldo;
  p.act = a->act;
  p.res_op = a->res_op;
  return STRATA_HIP_OK;
}

// The large-tile kernel streams 64-wide K steps (the last one masked when K
// is not a multiple of 64) with 32-bit lane offsets inside a 256-row block:
// row strides small enough.
// Sets the tile counts; the persistent grid is one workgroup per CU (the
// 128 KiB ring admits one).
static bool gemm_big(GemmParams& p, dim3& grid) {
  if (!(256 * p.ldx * 2 + 4096 < (int64_t)OOB && 256 * p.ldw * 2 + 4096 < (int64_t)OOB)) return false;
  p.mt = (int)((p.M + 255) / 256);
  p.nt = (int)((p.N + 255) / 256);
  const int64_t total = (int64_t)p.mt * p.nt;
  const int cus = device_cus();
  grid = dim3((unsigned)(total < cus ? total : cus));
  return total <= 0x7fffffff;
}

}  // namespace strata

extern "C" int strata_hip_gemm_bias_act(const strata_hip_gemm_args* a, void* stream) {
  GemmParams p;
  if (const int rc = gemm_params(a, p)) return rc;
  if (a->m == 0 || a->n == 0) return STRATA_HIP_OK;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid;
  if (gemm_big(p, grid)) {
    switch (p.act) {
      case STRATA_HIP_ACT_GELU_TANH: launch_dma_act<STRATA_HIP_ACT_GELU_TANH>(p, grid, st); break;
      case STRATA_HIP_ACT_GELU_ERF: launch_dma_act<STRATA_HIP_ACT_GELU_ERF>(p, grid, st); break;
      case STRATA_HIP_ACT_SIGMOID: launch_dma_act<STRATA_HIP_ACT_SIGMOID>(p, grid, st); break;
      case STRATA_HIP_ACT_GELU_TANH_GRAD: launch_dma_act<STRATA_HIP_ACT_GELU_TANH_GRAD>(p, grid, st); break;
      case STRATA_HIP_ACT_SIGMOID_GRAD: launch_dma_act<STRATA_HIP_ACT_SIGMOID_GRAD>(p, grid, st); break;
      default: launch_dma_act<STRATA_HIP_ACT_NONE>(p, grid, st); break;
    }
    return check_launch("gemm_dma_kernel");
  }
  return launch_gemm<128, 128, 2, 2>(p, st);
}

extern "C" int strata_hip_gemm_gelu_save(const strata_hip_gemm_args* a, void* dact, void* stream) {
  GemmParams p;
  if (const int rc = gemm_params(a, p)) return rc;
  if (a->act != STRATA_HIP_ACT_GELU_TANH || a->residual)
    return fail(STRATA_HIP_EINVAL, "gemm_gelu_save: act must be GELU_TANH, with no residual");
  if (a->m == 0 || a->n == 0) return STRATA_HIP_OK;
  if (!dact || ((uintptr_t)dact & 7)) return fail(STRATA_HIP_EINVAL, "gemm_gelu_save: dact must be 8-byte aligned");
  p.out2 = (bf16*)dact;
  dim3 grid;
  if (!gemm_big(p, grid))
    return fail(STRATA_HIP_EUNSUPPORTED, "gemm_gelu_save: row strides too long for the large-tile kernel");
  if (p.K % 64)
    hipLaunchKernelGGL((gemm_dma_kernel<STRATA_HIP_ACT_GELU_TANH, RES_NONE_T, true, true>), grid, dim3(512), 0,
                       (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL((gemm_dma_kernel<STRATA_HIP_ACT_GELU_TANH, RES_NONE_T, true>), grid, dim3(512), 0,
                       (hipStream_t)stream, p);
  return check_launch("gemm_dma_kernel (gelu save)");
}

// ---------------------------------------------------------------------------
// Bias gradient of the GEMM backward: out[n] = sum over m of g[m, n].
// Pass 1: a workgroup takes BG_ROWS rows x 128 columns.  A lane holds 8
// consecutive columns (16-byte loads); the 16 lanes of a quarter-wave cover
// the 128 columns of one row, so one load instruction reads 4 rows (1 KiB) and
// each wave walks every 16th row from its own start.  The lanes' fp32 sums are
// combined across the wave's quarters with two xor shuffles and across the
// four waves in LDS in wave order, and written as the chunk's partial row.
// Pass 2: per column, the chunks' partial rows are added by four threads (each
// a fixed quarter of the chunks, in order) and the four sums in order.  The
// order of every addition is fixed by the shape, so the result is the same bit
// for bit on every call.
// ---------------------------------------------------------------------------
namespace strata {

constexpr int BG_ROWS = 1024;  // rows per chunk (one partial row of the workspace each)

__global__ __launch_bounds__(256) void bias_grad_partial_kernel(const bf16* __restrict__ g, float* __restrict__ part,
                                                                int64_t M, int64_t N, int64_t ldg) {
  __shared__ float red[4][128];
  const int wave = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
  const int q = lane >> 4;                        // quarter of the wave: its row offset
  const int cl = 8 * (lane & 15);                 // first of the lane's 8 columns in the block
  const int64_t col = (int64_t)blockIdx.x * 128 + cl;
  const int64_t chunk = blockIdx.y;
  const int64_t r1 = min((chunk + 1) * (int64_t)BG_ROWS, M);
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (col < N) {
    int64_t r = chunk * BG_ROWS + 4 * wave + q;  // rows r, r + 16, ...
    const bf16* p = g + r * ldg + col;
    for (; r + 7 * 16 < r1; r += 8 * 16, p += 8 * 16 * ldg) {
      u32x4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = *(const u32x4*)(p + i * 16 * ldg);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          s[2 * w] += bf16_lo(v[i][w]);
          s[2 * w + 1] += bf16_hi(v[i][w]);
        }
    }
    for (; r < r1; r += 16, p += 16 * ldg) {
      const u32x4 v = *(const u32x4*)p;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        s[2 * w] += bf16_lo(v[w]);
        s[2 * w + 1] += bf16_hi(v[w]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    s[e] += __shfl_xor(s[e], 16);
    s[e] += __shfl_xor(s[e], 32);
  }
  if (q == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[wave][cl + e] = s[e];
  }
  __syncthreads();
  if (wave == 0 && q == 0 && col < N) {
    float t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = ((red[0][cl + e] + red[1][cl + e]) + red[2][cl + e]) + red[3][cl + e];
    float* o = part + chunk * N + col;
    *(f32x4*)o = (f32x4){t[0], t[1], t[2], t[3]};
    *(f32x4*)(o + 4) = (f32x4){t[4], t[5], t[6], t[7]};
  }
}

// 64 columns per workgroup; thread (w, c) adds chunks [w * per, (w + 1) * per)
// of column c, eight loads in flight, in chunk order.
__global__ __launch_bounds__(256) void bias_grad_finish_kernel(const float* __restrict__ part, bf16* __restrict__ out,
                                                               int64_t N, int64_t chunks) {
  __shared__ float red[4][64];
  const int w = (int)(threadIdx.x >> 6), c = (int)(threadIdx.x & 63);
  const int64_t col = (int64_t)blockIdx.x * 64 + c;
  const int64_t per = (chunks + 3) / 4;
  const int64_t c0 = min(w * per, chunks), c1 = min(c0 + per, chunks);
  float s = 0.f;
  if (col < N) {
    int64_t k = c0;
    for (; k + 8 <= c1; k += 8) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = part[(k + i) * N + col];
#pragma unroll
      for (int i = 0; i < 8; ++i) s += v[i];
    }
    for (; k < c1; ++k) s += part[k * N + col];
  }
  red[w][c] = s;
  __syncthreads();
  if (w == 0 && col < N) out[col] = (bf16)(((red[0][c] + red[1][c]) + red[2][c]) + red[3][c]);
}

static int64_t bias_grad_chunks(int64_t m) { return (m + BG_ROWS - 1) / BG_ROWS; }

}  // namespace strata

extern "C" int64_t strata_hip_bias_grad_workspace(int64_t m, int64_t n) {
  return m > 0 && n > 0 ? strata::bias_grad_chunks(m) * n : 0;
}

extern "C" int strata_hip_bias_grad(const strata_hip_bias_grad_args* a, void* stream) {
  using namespace strata;
  if (!a) return fail(STRATA_HIP_EINVAL, "bias_grad: null args");
  if (a->m < 0 || a->n < 0) return fail(STRATA_HIP_EINVAL, "bias_grad: bad m/n");
  if (a->n == 0) return STRATA_HIP_OK;
  if (!a->out || (a->m > 0 && (!a->g || !a->workspace))) return fail(STRATA_HIP_EINVAL, "bias_grad: null pointer");
  if (a->n % 8 || (a->m > 1 && (a->ldg < a->n || a->ldg % 8)) || ((uintptr_t)a->g & 15) || ((uintptr_t)a->workspace & 15))
    return fail(STRATA_HIP_EINVAL,
                "bias_grad: n and the row stride must be multiples of 8 (stride >= n), g and workspace 16-byte aligned");
  const int64_t chunks = bias_grad_chunks(a->m);
  const int64_t cblocks = (a->n + 127) / 128;
  if (chunks > 65535 || cblocks > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "bias_grad: too many rows");
  hipStream_t st = (hipStream_t)stream;
  if (a->m > 0)
    hipLaunchKernelGGL(bias_grad_partial_kernel, dim3((unsigned)cblocks, (unsigned)chunks), dim3(256), 0, st,
                       (const bf16*)a->g, a->workspace, a->m, a->n, a->m > 1 ? a->ldg : a->n);
  hipLaunchKernelGGL(bias_grad_finish_kernel, dim3((unsigned)((a->n + 63) / 64)), dim3(256), 0, st,
                     (const float*)a->workspace, (bf16*)a->out, a->n, a->m > 0 ? chunks : 0);
  return check_launch("bias_grad kernels");
}
