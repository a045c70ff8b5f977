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

  // state rows (c, dz, dy) -> tile[token][element], normalised, in bf16: a
  // wave per row, a lane per x (run <= 64)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int t = lane / p.px, dx = lane - t * p.px;
  for (int r = wave; r < rows; r += PIPE_THREADS / 64) {
    const int dy = r % p.py, dz = (r / p.py) % p.pz, c = r / (p.py * p.pz);
    if (lane < run) {
      const int64_t src = (((int64_t)b * p.C + c) * p.Z + (tz * p.pz + dz)) * (int64_t)p.Y * p.X +
                          (int64_t)(ty * p.py + dy) * p.X + x0 + lane;
      const float v = p.state[src];
      float n = v;
      if (p.mean) n = (v - p.mean[c]) / p.std[c];
      if (!__builtin_isfinite(v)) n = 0.f;
      tile[t * K + token_elem(p, 0, c, dz, dy, dx)] = (bf16)n;
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
  // tile -> state rows (c, dz, dy): a wave per row, a lane per x (run <= 64)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int t = lane / p.px, dx = lane - t * p.px;
  for (int r = wave; r < rows; r += PIPE_THREADS / 64) {
    const int dy = r % p.py, dz = (r / p.py) % p.pz, c = r / (p.py * p.pz);
    if (lane >= run) continue;
    const int xi = lane;
    const float pr = (float)tile[t * K + token_elem(p, p.order, c, dz, dy, dx)];
    // denormalise in fp32 (a multiply, then an add, each rounded: the pragma
    // above keeps them from contracting to an fma), round to bf16
    float d = pr;
    if (p.mean) d = pr * p.std[c] + p.mean[c];
    d = (float)(bf16)d;
    const int64_t sp = (int64_t)(tz * p.pz + dz) * p.Y * p.X + (int64_t)(ty * p.py + dy) * p.X + x0 + xi;
    const int sc = p.src ? p.src[c] : c;  // entries outside [0, Cin) add nothing
    if (sc >= 0 && sc < p.Cin) d += p.state[((int64_t)b * p.Cin + sc) * p.Z * (int64_t)p.Y * p.X + sp];
    if (p.clamp) {
      const float lo = p.clamp[c];
      if (!__builtin_isnan(lo)) d = d < lo ? lo : d;  // clamp(min=lo): NaN stays NaN
    }
    p.next[((int64_t)b * p.C + c) * p.Z * (int64_t)p.Y * p.X + sp] = d;
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

}  // namespace strata

using namespace strata;

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
