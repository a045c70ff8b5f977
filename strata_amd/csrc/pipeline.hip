// Rollout step around the network, for gfx950 (bandwidth-bound gathers).
//
// state_patchify: fp32 state [B, C, Z, Y, X] -> bf16 tokens [B, Tz, Ty, Tx, C*P]
//   (P = pz*py*px), the input normalisation of the pipeline
//   (screamcast/normalization.py:109-123) fused with the patchify of a
//   Conv3d(kernel = stride = patch) patch embedding.
// state_update: bf16 tokens [B, Tz, Ty, Tx, C*P] -> fp32 state [B, C, Z, Y, X],
//   the target denormalisation (normalization.py:102-107) and the mixed
//   state / difference update with the qv floor of MixedPredictionAsymmetric.step
//   (screamcast/model_pipelines.py:631-676).
//
// Both are transposes between the channels-first state and the channels-last
// tokens.  A workgroup takes NX consecutive tokens of one (b, tz, ty) token
// row, i.e. the x range [NX*px*xb, NX*px*(xb + 1)) of the C*pz*py state rows
// under them: state rows are read (or written) as runs of NX*px contiguous
// floats, the NX tokens as one contiguous run of NX*C*P bf16, and LDS holds the
// tokens in their final layout in between.
#include "common.h"

namespace strata {

struct PipeParams {
  const float* state;
  void* tokens;  // bf16, read by state_update
  float* next;
  const float* mean;
  const float* std;
  const int32_t* src;
  const float* clamp;
  int B, C, Cin, Z, Y, X;
  int pz, py, px, Tz, Ty, Tx;
  int order;  // element order within a token (state_update)
  int NX;     // tokens per workgroup
  int nxb;    // workgroups per token row
  int vec;    // token runs move as 4-byte pairs (even C*P, 4-byte aligned tokens)
};

constexpr int PIPE_LDS = 48 * 1024;
constexpr int PIPE_THREADS = 256;
constexpr int PIPE_U = 4;  // state-row passes per wave whose loads are in flight together

// Lanes a state-row run of `run` floats takes: run rounded up to a power of two (<= 64).
__device__ __forceinline__ int run_lanes(int run) {
  int l = 1;
  while (l < run) l <<= 1;
  return l;
}

// Element index of (c, dz, dy, dx) within a token.
__device__ __forceinline__ int token_elem(const PipeParams& p, int order, int c, int dz, int dy, int dx) {
  return order == 0 ? ((c * p.pz + dz) * p.py + dy) * p.px + dx : ((dz * p.py + dy) * p.px + dx) * p.C + c;
}

// Copy n bf16 between a token run in global memory and the LDS tile: 16-byte
// pieces when the run is 16-byte aligned and n a multiple of 8, else 4-byte
// pieces when p.vec allows, else single elements.
template <bool TO_LDS>
__device__ __forceinline__ void copy_run(const PipeParams& p, bf16* tile, bf16* g, int n, int tid) {
  if (((uintptr_t)g & 15u) == 0 && (n & 7) == 0) {
    u32x4* t = (u32x4*)tile;
    u32x4* q = (u32x4*)g;
    for (int i = tid; i < n / 8; i += PIPE_THREADS) {
      if (TO_LDS) t[i] = q[i];
      else q[i] = t[i];
    }
  } else if (p.vec) {
    uint32_t* t = (uint32_t*)tile;
    uint32_t* q = (uint32_t*)g;
    for (int i = tid; i < n / 2; i += PIPE_THREADS) {
      if (TO_LDS) t[i] = q[i];
      else q[i] = t[i];
    }
  } else {
    for (int i = tid; i < n; i += PIPE_THREADS) {
      if (TO_LDS) tile[i] = g[i];
      else g[i] = tile[i];
    }
  }
}

__global__ __launch_bounds__(PIPE_THREADS) void state_patchify_kernel(PipeParams p) {
  extern __shared__ __attribute__((aligned(16))) bf16 tile[];  // NX tokens, pipe_lds_bytes(p)
  int w = (int)blockIdx.x;
  const int xb = w % p.nxb;
  w /= p.nxb;
  const int ty = w % p.Ty;
  w /= p.Ty;
  const int tz = w % p.Tz;
  const int b = w / p.Tz;
  const int P = p.pz * p.py * p.px;
  const int K = p.C * P;
  const int tx0 = xb * p.NX;
  const int nt = min(p.NX, p.Tx - tx0);  // tokens of this workgroup
  const int run = nt * p.px;             // floats per state row
  const int rows = p.C * p.pz * p.py;
  const int x0 = tx0 * p.px;
  const int tid = (int)threadIdx.x;

  // state rows (c, dz, dy) -> tile[token][element], normalised, in bf16.  A
  // row's run takes RP lanes (run rounded up to a power of two), so a wave pass
  // covers 64 / RP rows, and a wave issues PIPE_U passes' loads before using them.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int RP = run_lanes(run), sub = lane / RP, xi = lane - sub * RP;
  const int t = xi / p.px, dx = xi - t * p.px;
  const int step = (PIPE_THREADS / 64) * (64 / RP);  // rows per pass of the workgroup
  for (int r0 = wave * (64 / RP) + sub; r0 < rows + step * (PIPE_U - 1); r0 += step * PIPE_U) {
    float v[PIPE_U];
    int cc[PIPE_U], el[PIPE_U];
#pragma unroll
    for (int u = 0; u < PIPE_U; ++u) {
      const int r = r0 + u * step;
      v[u] = 0.f;
      cc[u] = -1;
      if (r < rows && xi < run) {
        const int dy = r % p.py, dz = (r / p.py) % p.pz, c = r / (p.py * p.pz);
        cc[u] = c;
        el[u] = t * K + token_elem(p, 0, c, dz, dy, dx);
        v[u] = p.state[(((int64_t)b * p.C + c) * p.Z + (tz * p.pz + dz)) * (int64_t)p.Y * p.X +
                       (int64_t)(ty * p.py + dy) * p.X + x0 + xi];
      }
    }
#pragma unroll
    for (int u = 0; u < PIPE_U; ++u) {
      if (cc[u] >= 0) {
        float n = v[u];
        if (p.mean) n = (v[u] - p.mean[cc[u]]) / p.std[cc[u]];
        if (!__builtin_isfinite(v[u])) n = 0.f;
        tile[el[u]] = (bf16)n;
      }
    }
  }
  __syncthreads();
  // tile -> nt contiguous tokens
  bf16* dst = (bf16*)p.tokens + ((((int64_t)b * p.Tz + tz) * p.Ty + ty) * p.Tx + tx0) * K;
  copy_run<false>(p, tile, dst, nt * K, tid);
}

__global__ __launch_bounds__(PIPE_THREADS) void state_update_kernel(PipeParams p) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) bf16 tile[];  // NX tokens, pipe_lds_bytes(p)
  int w = (int)blockIdx.x;
  const int xb = w % p.nxb;
  w /= p.nxb;
  const int ty = w % p.Ty;
  w /= p.Ty;
  const int tz = w % p.Tz;
  const int b = w / p.Tz;
  const int P = p.pz * p.py * p.px;
  const int K = p.C * P;
  const int tx0 = xb * p.NX;
  const int nt = min(p.NX, p.Tx - tx0);
  const int run = nt * p.px;
  const int rows = p.C * p.pz * p.py;
  const int x0 = tx0 * p.px;
  const int tid = (int)threadIdx.x;

  // nt contiguous tokens -> tile
  bf16* src = (bf16*)p.tokens + ((((int64_t)b * p.Tz + tz) * p.Ty + ty) * p.Tx + tx0) * K;
  copy_run<true>(p, tile, src, nt * K, tid);
  __syncthreads();
  // tile -> state rows (c, dz, dy), as state_patchify: RP lanes per row, 64 / RP
  // rows per wave pass, PIPE_U passes' state loads issued before any store
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int RP = run_lanes(run), sub = lane / RP, xi = lane - sub * RP;
  const int t = xi / p.px, dx = xi - t * p.px;
  const int step = (PIPE_THREADS / 64) * (64 / RP);
  const int64_t plane = (int64_t)p.Z * p.Y * p.X;
  for (int r0 = wave * (64 / RP) + sub; r0 < rows + step * (PIPE_U - 1); r0 += step * PIPE_U) {
    float prev[PIPE_U];
    int cc[PIPE_U], el[PIPE_U];
    bool add[PIPE_U];
    int64_t sp[PIPE_U];
#pragma unroll
    for (int u = 0; u < PIPE_U; ++u) {
      const int r = r0 + u * step;
      prev[u] = 0.f;
      cc[u] = -1;
      add[u] = false;
      if (r < rows && xi < run) {
        const int dy = r % p.py, dz = (r / p.py) % p.pz, c = r / (p.py * p.pz);
        cc[u] = c;
        el[u] = t * K + token_elem(p, p.order, c, dz, dy, dx);
        sp[u] = (int64_t)(tz * p.pz + dz) * p.Y * p.X + (int64_t)(ty * p.py + dy) * p.X + x0 + xi;
        const int sc = p.src ? p.src[c] : c;  // entries outside [0, Cin) add nothing
        add[u] = sc >= 0 && sc < p.Cin;
        if (add[u]) prev[u] = p.state[((int64_t)b * p.Cin + sc) * plane + sp[u]];
      }
    }
#pragma unroll
    for (int u = 0; u < PIPE_U; ++u) {
      const int c = cc[u];
      if (c >= 0) {
        const float pr = (float)tile[el[u]];
        // denormalise in fp32 (a multiply, then an add, each rounded: the pragma
        // above keeps them from contracting to an fma), round to bf16
        float d = pr;
        if (p.mean) d = pr * p.std[c] + p.mean[c];
        d = (float)(bf16)d;
        if (add[u]) d += prev[u];
        if (p.clamp) {
          const float lo = p.clamp[c];
          if (!__builtin_isnan(lo)) d = d < lo ? lo : d;  // clamp(min=lo): NaN stays NaN
        }
        p.next[((int64_t)b * p.C + c) * plane + sp[u]] = d;
      }
    }
  }
}

// LDS of one workgroup: NX tokens of C*P bf16, rounded up to 16 bytes (sized
// to the need so that small tokens leave room for many workgroups per CU).
static size_t pipe_lds_bytes(const PipeParams& p) {
  return ((size_t)p.NX * p.C * p.pz * p.py * p.px * 2 + 15) / 16 * 16;
}

// Shared validation and launch geometry.  Returns OK and fills p, or an error.
static int pipe_setup(PipeParams& p, const char* name, int B, int C, const int32_t* grid, const int32_t* patch) {
  const std::string n(name);
  if (B < 0 || C <= 0) return fail(STRATA_HIP_EINVAL, n + ": bad batch/channels");
  static const char* axis = "zyx";
  for (int a = 0; a < 3; ++a) {
    if (grid[a] <= 0 || patch[a] <= 0)
      return fail(STRATA_HIP_EINVAL, n + ": grid and patch sizes must be positive on axis " + axis[a]);
    if (grid[a] % patch[a] != 0)
      return fail(STRATA_HIP_EINVAL, n + ": grid not a multiple of the patch on axis " + axis[a]);
  }
  p.B = B;
  p.C = C;
  p.Z = grid[0];
  p.Y = grid[1];
  p.X = grid[2];
  p.pz = patch[0];
  p.py = patch[1];
  p.px = patch[2];
  p.Tz = p.Z / p.pz;
  p.Ty = p.Y / p.py;
  p.Tx = p.X / p.px;
  const int64_t K = (int64_t)C * p.pz * p.py * p.px;
  if (K * 2 > PIPE_LDS)
    return fail(STRATA_HIP_EUNSUPPORTED, n + ": a token of C*pz*py*px elements must fit 48 KiB of bf16");
  if (p.px > 64) return fail(STRATA_HIP_EUNSUPPORTED, n + ": patch width above 64");
  // up to 64 state floats per row run (a lane each), as many tokens as LDS holds
  int NX = (int)(PIPE_LDS / (K * 2));
  const int nx_run = 64 / p.px > 1 ? 64 / p.px : 1;
  NX = NX < nx_run ? NX : nx_run;
  // at most 16 KiB when that still leaves 16 tokens: more workgroups per CU
  if (NX > 16 && (int64_t)NX * K * 2 > 16384) NX = (int)(16384 / (K * 2)) > 16 ? (int)(16384 / (K * 2)) : 16;
  NX = NX < p.Tx ? NX : p.Tx;
  p.NX = NX;
  p.nxb = (p.Tx + NX - 1) / NX;
  const int64_t blocks = (int64_t)B * p.Tz * p.Ty * p.nxb;
  if (blocks > 0x7fffffff || (int64_t)B * C * p.Z * p.Y * p.X > ((int64_t)1 << 40))
    return fail(STRATA_HIP_EUNSUPPORTED, n + ": problem too large for one launch");
  return STRATA_HIP_OK;
}

// One axis pass of the dealiasing low-pass (see strata_hip_dealias_axis).  The
// tensor is viewed as [outer, S, inner] around the filtered axis.  A wave owns
// DEALIAS_LPW lines and its lanes step through the lines' contiguous floats, so
// every index below the lane level is wave-uniform (scalar registers, no
// per-thread division), and the lines' loads of one tap are issued together:
//   x axis (inner = 1): a line is one row of S floats; output i of the row
//     reads its taps along the row;
//   y, z axes: a line is (o, i), the `inner` floats of output row i; its taps
//     are the rows clamp(P*(i/P) - lo + t, 0, S - P) + i%P of the same o.
struct DealiasParams {
  const float* src;
  float* dst;
  const float* mean;
  const float* std;
  int64_t lines;  // x: outer rows; y, z: outer * S
  int64_t inner;  // stride of the axis in floats
  int64_t cdiv;   // lines (x) or outer index (y, z) per channel step: c = (. / cdiv) % C
  int C, S, P, lo, taps;
  float f[16];
};

constexpr int DEALIAS_LPW = 8;  // lines per wave, their loads of one tap issued together

template <bool XAXIS>
__global__ __launch_bounds__(256) void dealias_axis_kernel(DealiasParams p) {
  constexpr int R = DEALIAS_LPW;
  const int64_t line0 = ((int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) * R;
  const int lane = threadIdx.x & 63;
  if (line0 >= p.lines) return;  // uniform per wave
  const float* src[R];
  float* dst[R];
  float m[R], sd[R];
  int j0[R], u[R];
  bool live[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t line = line0 + r < p.lines ? line0 + r : p.lines - 1;  // a repeated last line is harmless
    live[r] = line0 + r < p.lines;
    int64_t o = line;  // x: the row; y, z: the outer index
    int irow = 0;      // y, z: the output row
    if constexpr (!XAXIS) {
      o = line / p.S;
      irow = (int)(line - o * p.S);
    }
    m[r] = 0.f;
    sd[r] = 1.f;
    if (p.mean) {
      const int c = (int)((o / p.cdiv) % p.C);
      m[r] = p.mean[c];
      sd[r] = p.std[c];
    }
    if constexpr (XAXIS) {
      src[r] = p.src + line * p.S;
      dst[r] = p.dst + line * p.S;
    } else {
      j0[r] = p.P * (irow / p.P) - p.lo;
      u[r] = irow % p.P;
      src[r] = p.src + o * p.S * p.inner;
      dst[r] = p.dst + line * p.inner;
    }
  }
  const int64_t n = XAXIS ? p.S : p.inner;
  for (int64_t k = lane; k < n; k += 64) {
    int xj0 = 0, xu = 0;
    if constexpr (XAXIS) {
      xj0 = p.P * ((int)k / p.P) - p.lo;
      xu = (int)k % p.P;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    for (int t = 0; t < p.taps; ++t) {
      float v[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if constexpr (XAXIS)
          v[r] = src[r][min(max(xj0 + t, 0), p.S - p.P) + xu];
        else
          v[r] = src[r][(int64_t)(min(max(j0[r] + t, 0), p.S - p.P) + u[r]) * p.inner + k];
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float nv = v[r];
        if (p.mean) nv = (v[r] - m[r]) / sd[r];
        if (!__builtin_isfinite(v[r])) nv = 0.f;
        acc[r] = fmaf(p.f[t], nv, acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (live[r]) dst[r][k] = acc[r];
  }
}

}  // namespace strata

using namespace strata;

extern "C" int strata_hip_dealias_axis(const strata_hip_dealias_axis_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "dealias_axis: null args");
  if (!a->src || !a->dst) return fail(STRATA_HIP_EINVAL, "dealias_axis: null tensor pointer");
  if ((a->mean == nullptr) != (a->std == nullptr))
    return fail(STRATA_HIP_EINVAL, "dealias_axis: mean and std must both be given or both be NULL");
  if (a->batch < 0 || a->channels <= 0) return fail(STRATA_HIP_EINVAL, "dealias_axis: bad batch/channels");
  if (a->grid[0] <= 0 || a->grid[1] <= 0 || a->grid[2] <= 0) return fail(STRATA_HIP_EINVAL, "dealias_axis: bad grid");
  if (a->axis < 0 || a->axis > 2) return fail(STRATA_HIP_EINVAL, "dealias_axis: axis must be 0, 1 or 2");
  const int S = a->grid[a->axis];
  if (a->patch <= 0 || S % a->patch != 0)
    return fail(STRATA_HIP_EINVAL, "dealias_axis: patch must be positive and divide the grid on the axis");
  if (a->taps < 1 || a->taps > 16) return fail(STRATA_HIP_EINVAL, "dealias_axis: taps must be in 1..16");
  if (a->src == a->dst) return fail(STRATA_HIP_EINVAL, "dealias_axis: src and dst must not alias");
  DealiasParams p = {};
  p.src = a->src;
  p.dst = a->dst;
  p.mean = a->mean;
  p.std = a->std;
  p.C = a->channels;
  p.S = S;
  p.P = a->patch;
  p.taps = a->taps;
  p.lo = (a->taps - 1) / 2;
  for (int t = 0; t < a->taps; ++t) p.f[t] = a->filter[t];
  const int64_t Z = a->grid[0], Y = a->grid[1], X = a->grid[2];
  const int64_t total = (int64_t)a->batch * a->channels * Z * Y * X;
  if (total == 0) return STRATA_HIP_OK;
  if (total > ((int64_t)1 << 40)) return fail(STRATA_HIP_EUNSUPPORTED, "dealias_axis: problem too large");
  // [outer, S, inner] around the axis; cdiv: outer indices (y, z) or rows (x) per channel
  p.inner = a->axis == 2 ? 1 : (a->axis == 1 ? X : Y * X);
  const int64_t outer = total / (S * p.inner);
  p.lines = a->axis == 2 ? outer : outer * S;
  p.cdiv = a->axis == 0 ? 1 : (a->axis == 1 ? Z : Z * Y);
  const int64_t blocks = (p.lines + 4 * DEALIAS_LPW - 1) / (4 * DEALIAS_LPW);
  if (blocks > 0x7fffffff) return fail(STRATA_HIP_EUNSUPPORTED, "dealias_axis: problem too large for one launch");
  if (a->axis == 2)
    hipLaunchKernelGGL(dealias_axis_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(dealias_axis_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
  return check_launch("dealias_axis_kernel");
}

extern "C" int strata_hip_state_patchify(const strata_hip_state_patchify_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "state_patchify: null args");
  PipeParams p = {};
  const int rc = pipe_setup(p, "state_patchify", a->batch, a->channels, a->grid, a->patch);
  if (rc != STRATA_HIP_OK) return rc;
  if (!a->state || !a->tokens) return fail(STRATA_HIP_EINVAL, "state_patchify: null tensor pointer");
  if ((a->mean == nullptr) != (a->std == nullptr))
    return fail(STRATA_HIP_EINVAL, "state_patchify: mean and std must both be given or both be NULL");
  p.state = a->state;
  p.tokens = a->tokens;
  p.mean = a->mean;
  p.std = a->std;
  p.vec = (p.C * p.pz * p.py * p.px) % 2 == 0 && ((uintptr_t)a->tokens & 3u) == 0;
  const int64_t blocks = (int64_t)p.B * p.Tz * p.Ty * p.nxb;
  if (blocks == 0) return STRATA_HIP_OK;
  hipLaunchKernelGGL(state_patchify_kernel, dim3((unsigned)blocks), dim3(PIPE_THREADS), pipe_lds_bytes(p),
                     (hipStream_t)stream, p);
  return check_launch("state_patchify_kernel");
}

extern "C" int strata_hip_state_update(const strata_hip_state_update_args* a, void* stream) {
  if (!a) return fail(STRATA_HIP_EINVAL, "state_update: null args");
  PipeParams p = {};
  const int rc = pipe_setup(p, "state_update", a->batch, a->channels, a->grid, a->patch);
  if (rc != STRATA_HIP_OK) return rc;
  if (!a->pred || !a->next) return fail(STRATA_HIP_EINVAL, "state_update: null tensor pointer");
  if (a->order != 0 && a->order != 1) return fail(STRATA_HIP_EINVAL, "state_update: order must be 0 or 1");
  if ((a->mean == nullptr) != (a->std == nullptr))
    return fail(STRATA_HIP_EINVAL, "state_update: mean and std must both be given or both be NULL");
  // Without a channel map every channel is a difference of the same state channel.
  if (!a->src_channel && a->state_channels < a->channels)
    return fail(STRATA_HIP_EINVAL, "state_update: state has fewer channels than the prediction");
  if (a->state_channels < 0 || (a->state_channels > 0) != (a->state != nullptr))
    return fail(STRATA_HIP_EINVAL, "state_update: state and state_channels must both be given or both be empty");
  p.tokens = const_cast<void*>(a->pred);
  p.state = a->state;
  p.next = a->next;
  p.mean = a->mean;
  p.std = a->std;
  p.src = a->src_channel;
  p.clamp = a->clamp_min;
  p.Cin = a->state_channels;
  p.order = a->order;
  p.vec = (p.C * p.pz * p.py * p.px) % 2 == 0 && ((uintptr_t)a->pred & 3u) == 0;
  const int64_t blocks = (int64_t)p.B * p.Tz * p.Ty * p.nxb;
  if (blocks == 0) return STRATA_HIP_OK;
  hipLaunchKernelGGL(state_update_kernel, dim3((unsigned)blocks), dim3(PIPE_THREADS), pipe_lds_bytes(p),
                     (hipStream_t)stream, p);
  return check_launch("state_update_kernel");
}
