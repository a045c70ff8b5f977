/*
 * strata_hip.h — C ABI of the MI355X (gfx950) kernels for the Strata
 * transformer block's hot path: 3D neighbourhood attention (NA3D), the
 * stereographic-RoPE + QKV-pack prologue, the bias/GELU/residual GEMM and the
 * non-affine LayerNorm; around it, the cube-sphere halo fill and the rollout
 * step's state normalisation / patchify and state update, and the NA3D backward.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers owned by the caller.  Every kernel is
 *     hand-written; the library allocates and frees no device memory, keeps no
 *     state between calls and links no library beyond the HIP runtime.
 *   - `stream` is a hipStream_t (passed as void* so that the header needs no
 *     HIP include).  Work is enqueued asynchronously on that stream; there is
 *     no device synchronisation inside the library.
 *   - Return value: STRATA_HIP_OK (0) or a negative STRATA_HIP_E* code.  The
 *     message of the last failure on the calling thread is returned by
 *     strata_hip_last_error().
 *   - Token tensors use the heads-last layout [B, Z, Y, X, H, D] (NATTEN >= 0.20
 *     layout).  Strides are in ELEMENTS over (b, z, y, x, h); the d stride is 1.
 */
#ifndef STRATA_HIP_H
#define STRATA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STRATA_HIP_ABI_VERSION 6

enum strata_hip_status {
  STRATA_HIP_OK = 0,
  STRATA_HIP_EINVAL = -1,      /* bad shape, stride, kernel size or pointer */
  STRATA_HIP_EUNSUPPORTED = -2, /* valid request this build has no kernel for */
  STRATA_HIP_ELAUNCH = -3       /* hipLaunchKernel / hipGetLastError failure */
};

enum strata_hip_dtype { STRATA_HIP_F32 = 0, STRATA_HIP_BF16 = 1 };

enum strata_hip_act {
  STRATA_HIP_ACT_NONE = 0,
  STRATA_HIP_ACT_GELU_TANH = 1,
  STRATA_HIP_ACT_GELU_ERF = 2,
  STRATA_HIP_ACT_SIGMOID = 3,       /* the attention gate */
  STRATA_HIP_ACT_GELU_TANH_GRAD = 4, /* d/dx GELU(tanh): with res_op MUL and residual = the upstream
                                        gradient, the MLP backward's gradient at fc1's output */
  STRATA_HIP_ACT_SIGMOID_GRAD = 5     /* d/dx sigmoid: the gate's backward (res_op MUL) */
};
/* How the GEMM epilogue combines act(x @ w^T + bias) with `residual`. */
enum strata_hip_res_op { STRATA_HIP_RES_ADD = 0, STRATA_HIP_RES_MUL = 1 };

enum strata_hip_rope_layout {
  STRATA_HIP_ROPE_HALF = 0,       /* pair p = (d=p, d=p+D/2)   ("rotate_half") */
  STRATA_HIP_ROPE_INTERLEAVED = 1 /* pair p = (d=2p, d=2p+1) */
};

/* ---------------------------------------------------------------------------
 * NA3D forward.
 * Replaces natten.na3d(query, key, value, kernel_size, stride=1, dilation,
 * is_causal=False, scale) of NATTEN 0.21.5 (pinned at
 * docker/build_natten.sh:21 and Makefile:11; reached through the backend
 * string of screamcast/config.py:99 -> train.py:143 ->
 * screamcast/strata_wrappers.py:331,490,582).
 *
 * q, k, v share the token grid `grid` = (Z, Y, X).  Only the queries inside
 * the box [q_origin, q_origin + q_extent) are computed; `out` has the box's
 * shape [B, Ez, Ey, Ex, H, D].  Windows are NATTEN's clamped windows on the
 * full grid, so out == natten.na3d(q, k, v)[:, box].  Per axis: odd kernel
 * k, dilation d with d*k <= L; a query i with g = i mod d attends keys
 * g + d*(s + [0, k)), s = clamp(i/d - k/2, 0, ceil((L-g)/d) - k).
 * bf16 inputs: fp32 accumulation and softmax, bf16 output.  f32 inputs: f32.
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_na3d_args {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int32_t dtype;       /* strata_hip_dtype, same for q, k, v, out */
  int32_t batch;
  int32_t heads;
  int32_t head_dim;
  int32_t grid[3];     /* Z, Y, X of the q/k/v token grid */
  int32_t q_origin[3]; /* first query (z, y, x) of the output box */
  int32_t q_extent[3]; /* output box size (Ez, Ey, Ex) */
  int32_t kernel[3];   /* window (kz, ky, kx), odd */
  int32_t dilation[3];
  int32_t reserved;
  float scale;         /* softmax scale, usually head_dim^-1/2 */
  float reserved_f;
  int64_t q_stride[5]; /* element strides over (b, z, y, x, h) */
  int64_t k_stride[5];
  int64_t v_stride[5];
  int64_t o_stride[5]; /* strides of `out` over (b, z', y', x', h) */
  float* lse;          /* fp32 [B, Z', Y', X', H] contiguous, or NULL: each query's
                          log2-sum-exp over its window of the log2-unit scores
                          scale*log2(e)*q.k (q rounded to bf16 after the scaling on
                          the bf16 path), the statistic strata_hip_na3d_bwd needs */
} strata_hip_na3d_args;

int strata_hip_na3d_fwd(const strata_hip_na3d_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * NA3D forward with the queries' rotary embedding applied inside the kernel.
 * Replaces the query half of the attention forward's RoPE followed by
 * natten.na3d (screamcast/strata_wrappers.py:331-338, the stereographic RoPE
 * helpers imported at :52): q is the UNROTATED query (e.g. a strided view of
 * the qkv projection's output), k already rotated (strata_hip_rope_qkv_pack
 * with q = NULL), and the result equals strata_hip_na3d_fwd on
 * q' = rope(q), q' rounded to bf16 as the pack rounds it.  Half layout only
 * (pair j = (j, j + 32)); cos, sin: fp32 [B, table_z, Y, X, 32] contiguous,
 * 16-byte aligned, indexed by each query's full-grid position; table_z = 1
 * (broadcast over z) or Z.  bf16, head_dim 64, args->lse must be NULL (the
 * backward needs the rotated q: training keeps the pack).  Windows and
 * layouts that run the wide-window strip kernels (kx 10-13, ky 13) return
 * STRATA_HIP_EUNSUPPORTED; strata_hip_na3d_fwd_rope_q_supported() answers the
 * same question without launching (1 = supported, 0 = not).
 * ------------------------------------------------------------------------- */
int strata_hip_na3d_fwd_rope_q(const strata_hip_na3d_args* args, const float* cos, const float* sin, int32_t table_z,
                               void* stream);
int strata_hip_na3d_fwd_rope_q_supported(const strata_hip_na3d_args* args, const float* cos, const float* sin,
                                         int32_t table_z);

/* ---------------------------------------------------------------------------
 * NA3D backward: dq, dk, dv of natten.na3d for out = na3d(q, k, v) over the
 * whole grid (the autograd function of NATTEN 0.21.5 that training reaches
 * through train.py:1161), same windows, kernel, dilation and scale as the
 * forward.  q, k, v, out, dout, dq, dk, dv: contiguous heads-last
 * [B, Z, Y, X, H, D], one dtype (f32 or bf16; fp32 math), 16-byte aligned;
 * head_dim 32, 64 or 128.  workspace: 2 * B*Z*Y*X*H floats of caller memory
 * (per-query log-sum-exp and rowsum(dout * out)), overwritten.  lse: the
 * forward's lse output for the same q, k (strata_hip_na3d_fwd over the whole
 * grid), or NULL; given, the log-sum-exp is not recomputed (only the rowsum
 * half of the workspace is written).
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_na3d_bwd_args {
  const void* q;
  const void* k;
  const void* v;
  const void* out;  /* the forward's output */
  const void* dout; /* gradient of the loss w.r.t. out */
  void* dq;
  void* dk;
  void* dv;
  float* workspace;
  int32_t dtype;
  int32_t batch;
  int32_t heads;
  int32_t head_dim;
  int32_t grid[3];
  int32_t kernel[3];
  int32_t dilation[3];
  float scale;
  const float* lse; /* [B, Z, Y, X, H] from the forward, or NULL */
} strata_hip_na3d_bwd_args;

int strata_hip_na3d_bwd(const strata_hip_na3d_bwd_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * NA3D backward without allocation: no counterpart in the reference.  For
 * callers that cannot allocate device memory or pass a workspace (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as strata_hip_na3d_bwd, except that `workspace` must
 * be NULL: the per-query statistics live in a scratch array of the library's
 * own, one per device (16 MiB, held until the process ends), so at most
 * B*Z*Y*X*H = 2^21 (query, head) pairs per call; larger calls return
 * STRATA_HIP_EUNSUPPORTED.  Nothing is allocated or freed.  Every call on one
 * device uses that device's scratch: calls that overlap in time on one device
 * (different streams or threads) race.
 * ------------------------------------------------------------------------- */
int strata_hip_na3d_bwd_noalloc(const strata_hip_na3d_bwd_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Stereographic-RoPE + QKV pack.
 * Replaces the attention's qkv split + RoPE of the physicsnemo Strata block
 * (attn.qkv keys at tests/regression_data/sweep1_...param_order.txt:3-4;
 * RoPE helpers imported at screamcast/strata_wrappers.py:52, base and length
 * scale set at :333-338).
 *
 * qkv: [M, 3*H*D] bf16, row stride `qkv_row_stride` elements, column order
 * (3, H, D) (nn.Linear output of attn.qkv).  M = B*Z*Y*X tokens.
 * cos/sin: f32 tables [B, Zt, Y, X, D/2] contiguous, Zt in {1, Z} (Zt = 1
 * broadcasts one table over all levels).
 * q, k, v: [M, H, D] bf16 contiguous (heads-last token layout).  RoPE rotates
 * the pairs of q and k; v is copied.  Any of q/k/v may alias nothing else.
 * v may be NULL: then only q and k are written (a caller that reads v straight
 * out of qkv, as a view with token stride qkv_row_stride, saves the copy).
 * q may be NULL too: then only k (and v) are written, for a caller that
 * rotates the queries inside NA3D (strata_hip_na3d_fwd_rope_q).
 *
 * qk_norm = 1 applies RMSNorm over D to every (token, head) of q and k before
 * the rotation, x * rsqrt(mean(x^2) + qk_norm_eps) * weight (fp32 math;
 * weight bf16 [D], or NULL for no elementwise affine): the block's optional
 * qk normalisation (screamcast/config.py:91-93 qk_norm /
 * qk_norm_elementwise_affine, passed at screamcast/strata_wrappers.py:324-325).
 * It needs D/16 (half layout) or D/8 (interleaved) to be a power of two.
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_rope_pack_args {
  const void* qkv;
  const float* cos;
  const float* sin;
  void* q;
  void* k;
  void* v;
  int32_t batch;
  int32_t grid[3];    /* Z, Y, X */
  int32_t table_z;    /* Zt: 1 or Z */
  int32_t heads;
  int32_t head_dim;
  int32_t layout;     /* strata_hip_rope_layout */
  int64_t qkv_row_stride;
  int32_t qk_norm;    /* 0: off, 1: RMSNorm of q and k per (token, head) */
  float qk_norm_eps;
  const void* q_norm_weight; /* bf16 [D] or NULL */
  const void* k_norm_weight; /* bf16 [D] or NULL */
} strata_hip_rope_pack_args;

int strata_hip_rope_qkv_pack(const strata_hip_rope_pack_args* args, void* stream);

/* Backward of the pack: dqkv [M, (3, H, D)] (row stride dqkv_row_stride) =
 * (R(-theta) dq, R(-theta) dk, dv) for dq, dk, dv [M, H, D] contiguous bf16
 * and the forward's cos/sin tables and layout.  dv may be NULL: v's columns of
 * dqkv are then written as zeros (a v read as a view of qkv adds its gradient
 * there itself).  With qk_norm = 1 the q and k
 * columns are further taken through the RMSNorm backward, recomputed from the
 * forward's input qkv (row stride qkv_row_stride):
 *   g = R(-theta) dout * w,  r = 1/sqrt(mean(x^2) + eps),
 *   dx = r * g - x * r^3 * <g, x> / D,
 * and, for a weight given (q_norm_weight / k_norm_weight, bf16 [D]), the
 * weight gradient sum over tokens and heads of (R(-theta) dout) * x * r is
 * ADDED to dq_norm_weight / dk_norm_weight (fp32 [D]; the caller zeroes them;
 * the sum is accumulated with atomics, so its rounding order varies).
 * Backward of the forward strata_hip_rope_qkv_pack with the same
 * qk_norm / qk_norm_eps / weights. */
typedef struct strata_hip_rope_pack_bwd_args {
  const void* dq;
  const void* dk;
  const void* dv;
  const float* cos;
  const float* sin;
  void* dqkv;
  int32_t batch;
  int32_t grid[3];
  int32_t table_z;
  int32_t heads;
  int32_t head_dim;
  int32_t layout;
  int64_t dqkv_row_stride;
  const void* qkv;           /* forward input [M, (3, H, D)] bf16; read only with qk_norm */
  int64_t qkv_row_stride;
  const void* q_norm_weight; /* bf16 [D] or NULL */
  const void* k_norm_weight; /* bf16 [D] or NULL */
  float* dq_norm_weight;     /* fp32 [D], accumulated; NULL iff q_norm_weight is NULL */
  float* dk_norm_weight;     /* fp32 [D], accumulated; NULL iff k_norm_weight is NULL */
  int32_t qk_norm;           /* 0 or 1, as in the forward */
  float qk_norm_eps;
} strata_hip_rope_pack_bwd_args;

int strata_hip_rope_qkv_pack_bwd(const strata_hip_rope_pack_bwd_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * GEMM with fused epilogue:  out = act(x @ w^T + bias) (+ or *) residual
 * Replaces nn.Linear (+ GELU) of the block: attn.qkv, attn.proj and the Mlp
 * fc1 -> GELU(tanh) -> fc2 chain (Mlp layers.0 / layers.2 at
 * screamcast/checkpoint_compat.py:243-249; tanh GELU forced by
 * screamcast/strata_wrappers.py:76-100), and the gated-attention gate
 * a * sigmoid(gate_proj(x)) (attn.gate_proj in the manifests,
 * tests/regression_data/sweep1_...param_order.txt:7-8): act = SIGMOID,
 * res_op = MUL, residual = the attention output a.
 *
 * x: [M, K] bf16 (row stride ldx), w: [N, K] bf16 (nn.Linear layout, row
 * stride ldw), bias: [N] bf16 or NULL, residual: [M, N] bf16 (row stride ldr)
 * or NULL, out: [M, N] bf16 (row stride ldo).  fp32 accumulation.  The
 * residual is added (res_op ADD) or multiplied (res_op MUL) after the
 * activation.  K must be a multiple of 8, every row stride a multiple of 8
 * elements, x, w, out and residual 16-byte aligned and bias 8-byte aligned
 * (STRATA_HIP_EINVAL otherwise).  `out` may alias `residual`.
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_gemm_args {
  const void* x;
  const void* w;
  const void* bias;
  const void* residual;
  void* out;
  int64_t m;
  int64_t n;
  int64_t k;
  int64_t ldx;
  int64_t ldw;
  int64_t ldr;
  int64_t ldo;
  int32_t act;    /* strata_hip_act */
  int32_t res_op; /* strata_hip_res_op */
} strata_hip_gemm_args;

int strata_hip_gemm_bias_act(const strata_hip_gemm_args* args, void* stream);

/* fc1 -> GELU(tanh) for training (the Mlp of screamcast/checkpoint_compat.py:243-249
 * under loss.backward(), train.py:1161): strata_hip_gemm_bias_act with act =
 * GELU_TANH and no residual, and in the same launch dact = gelu'(x @ w^T + bias),
 * bf16 [M, N] with out's row stride ldo, the derivative the backward multiplies
 * by the upstream gradient (instead of recomputing the GEMM).  The argument
 * rules of strata_hip_gemm_bias_act apply (K a multiple of 8); row strides too
 * long for the large-tile kernel's 32-bit lane offsets (256 * ld * 2 bytes past
 * 2^31) return STRATA_HIP_EUNSUPPORTED (the caller then recomputes). */
int strata_hip_gemm_gelu_save(const strata_hip_gemm_args* args, void* dact, void* stream);

/* Bias gradient of the GEMM backward (nn.Linear's d bias: the output gradient
 * summed over rows, as torch autograd forms it when training reaches the
 * block's Linears through train.py:1161):  out[n] = sum_m g[m, n].
 * g: [M, N] bf16, row stride ldg (>= N; N and ldg multiples of 8 elements,
 * g 16-byte aligned); out: [N] bf16; workspace: fp32, 16-byte aligned, at
 * least strata_hip_bias_grad_workspace(M, N) elements (per-chunk partial
 * sums).  fp32 accumulation in an order fixed by the shape: the result repeats
 * bit for bit. */
typedef struct strata_hip_bias_grad_args {
  const void* g;
  void* out;
  float* workspace;
  int64_t m;
  int64_t n;
  int64_t ldg;
} strata_hip_bias_grad_args;

int64_t strata_hip_bias_grad_workspace(int64_t m, int64_t n);
int strata_hip_bias_grad(const strata_hip_bias_grad_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Non-affine LayerNorm over the last dimension (the block's two pre-norms,
 * which carry no parameters in the state-dict manifests
 * tests/regression_data/sweep1_...param_order.txt:3-12).
 * x, out: [M, C] bf16, row strides ldx / ldo elements; fp32 statistics.
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_layer_norm_args {
  const void* x;
  void* out;
  int64_t m;
  int64_t c;
  int64_t ldx;
  int64_t ldo;
  float eps;
  int32_t reserved;
} strata_hip_layer_norm_args;

int strata_hip_layer_norm(const strata_hip_layer_norm_args* args, void* stream);

/* Backward of the non-affine LayerNorm: dx from x and dy (all [M, C] bf16 with
 * one row stride `ld`), dx = rstd * (dy - mean(dy) - xh * mean(dy * xh)),
 * xh = (x - mean) * rstd, fp32 statistics recomputed from x. */
typedef struct strata_hip_layer_norm_bwd_args {
  const void* x;
  const void* dy;
  void* dx;
  int64_t m;
  int64_t c;
  int64_t ld;
  float eps;
  int32_t reserved;
} strata_hip_layer_norm_bwd_args;

int strata_hip_layer_norm_bwd(const strata_hip_layer_norm_bwd_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Cube-sphere halo fill: the single-GPU local counterpart of the rollout's
 * halo exchange, create_padded_faces_batched
 * (screamcast/cubesphere_transforms.py:369-445; neighbour table :149-196, edge
 * strips and quarter turns :199-273, corner fill :276-366).
 * src: [lead, 6, n, n], dst: [lead, 6, n + 2*pad, n + 2*pad], contiguous,
 * f32 or bf16 (strata_hip_dtype).  pad <= n; dst must not alias src.
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_cube_pad_args {
  const void* src;
  void* dst;
  int32_t dtype;
  int32_t face_size; /* n */
  int32_t pad;
  int32_t reserved;
  int64_t lead;      /* product of the leading dims */
} strata_hip_cube_pad_args;

int strata_hip_cube_pad_faces(const strata_hip_cube_pad_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Crop of padded tiles/faces: TileTopology.crop
 * (screamcast/distributed_halo.py:143-147).
 * src: [planes, extent, extent], dst: [planes, extent - 2*halo, extent - 2*halo],
 * contiguous, f32 or bf16.
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_cube_crop_args {
  const void* src;
  void* dst;
  int32_t dtype;
  int32_t extent; /* side of the padded square */
  int32_t halo;
  int32_t reserved;
  int64_t planes;
} strata_hip_cube_crop_args;

int strata_hip_cube_crop(const strata_hip_cube_crop_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Pipeline step, input side: the input normalisation of the model state
 * (RunningNorm2d.forward, screamcast/normalization.py:109-123, applied by
 * MixedPredictionAsymmetric.forward_from_flat, screamcast/model_pipelines.py:210-211)
 * fused with the patchify of a Conv3d(kernel = stride = patch) patch embedding:
 *   tok[b, t, e] = bf16((state[b, c, pz*tz + dz, py*ty + dy, px*tx + dx] - mean[c]) / std[c]),
 *                  0 where that state value is not finite,
 * token t = (tz, ty, tx) row-major over the token grid, element
 * e = ((c*pz + dz)*py + dy)*px + dx: the order of a Conv3d weight [E, C, pz, py, px]
 * flattened, so tok @ weight.reshape(E, -1)^T + bias is the patch embedding of
 * the normalised state.  std[c] = sqrt(var[c]) + eps, computed by the caller in
 * fp32 as normalization.py:117 does; mean and std NULL: no normalisation.
 * state: fp32 [B, C, Z, Y, X] contiguous; tok: bf16 [B, Z/pz, Y/py, X/px, C*pz*py*px]
 * contiguous; each grid size a multiple of its patch size.
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_state_patchify_args {
  const float* state;
  void* tokens;
  const float* mean; /* [C] or NULL */
  const float* std;  /* [C] or NULL (with mean) */
  int32_t batch;
  int32_t channels;  /* C */
  int32_t grid[3];   /* Z, Y, X of the state */
  int32_t patch[3];  /* pz, py, px */
} strata_hip_state_patchify_args;

int strata_hip_state_patchify(const strata_hip_state_patchify_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Dealiased patch embedding (DealiasedPatchEmbed3D, screamcast/dealias.py:28-143):
 * a stride-1 valid Conv3d (kernel = patch) followed by a per-axis low-pass,
 * replicate-padded by (k-1)/2 below and the rest above, decimated by the patch
 * stride.  Both stages are linear and each axis filter sums to 1, so the
 * embedding equals the plain patch embedding (state_patchify + GEMM with the
 * same proj weight and bias) of the state filtered, per decimated axis, as
 *   dst[.., i, ..] = sum_{t < taps} filter[t] *
 *                    n(src[.., clamp(p*(i/p) - lo + t, 0, S - p) + i % p, ..])
 * with S the grid size and p the patch size on that axis, lo = (taps - 1) / 2,
 * and n(v) = (v - mean[c]) / std[c] (0 for non-finite v) when mean/std are
 * given (the input normalisation, fused into the first pass), else v.
 * src, dst: fp32 [B, C, Z, Y, X] contiguous, not aliased.  filter: the axis
 * taps already divided by their sum (the reference's dealias_filter is their
 * outer product over the axes); axes with patch 1 take no pass.
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_dealias_axis_args {
  const float* src;
  float* dst;
  const float* mean; /* [C] or NULL */
  const float* std;  /* [C] or NULL (with mean) */
  int32_t batch;
  int32_t channels;
  int32_t grid[3];   /* Z, Y, X */
  int32_t axis;      /* 0: Z, 1: Y, 2: X */
  int32_t patch;     /* patch size along the axis, divides grid[axis] */
  int32_t taps;      /* 1..16 */
  float filter[16];
} strata_hip_dealias_axis_args;

int strata_hip_dealias_axis(const strata_hip_dealias_axis_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Pipeline step, output side: unpatchify of the prediction tokens, the target
 * denormalisation (RunningNorm2d.denormalize, screamcast/normalization.py:102-107)
 * and the prognostic state update of MixedPredictionAsymmetric.step
 * (screamcast/model_pipelines.py:631-662, _process_mixed_statediff_predictions :664-676):
 *   d = bf16(pred * std[c] + mean[c])            (fp32 multiply, then add, then bf16)
 *   next[b, c, z, y, x] = d + state[b, src[c], z, y, x]   src[c] >= 0: difference prediction
 *                       = d                               src[c] <  0: state prediction
 *   then max(next, clamp_min[c]) where clamp_min[c] is not NaN (the qv floor, :652-658).
 * pred: bf16 [B, Z/pz, Y/py, X/px, C*pz*py*px] contiguous, element order
 *   order 0: ((c*pz + dz)*py + dy)*px + dx   (Conv3d / ConvTranspose3d weight order)
 *   order 1: ((dz*py + dy)*px + dx)*C + c     (patch-major, channels last)
 * state: fp32 [B, Cin, Z, Y, X] contiguous; next: fp32 [B, C, Z, Y, X] contiguous.
 * NULL tables: mean 0, std 1, src[c] = c (every channel a difference), no clamp.
 * src[c] outside [0, Cin) adds nothing; state may be NULL with state_channels 0
 * (every channel a state prediction).  next may alias state only when every
 * src[c] is c or negative.
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_state_update_args {
  const void* pred;
  const float* state;
  float* next;
  const float* mean;          /* [C] or NULL */
  const float* std;           /* [C] or NULL */
  const int32_t* src_channel; /* [C] or NULL */
  const float* clamp_min;     /* [C] or NULL */
  int32_t batch;
  int32_t channels;           /* C of pred and next */
  int32_t state_channels;     /* Cin of state */
  int32_t order;              /* 0 or 1, see above */
  int32_t grid[3];            /* Z, Y, X of the state */
  int32_t patch[3];           /* pz, py, px */
} strata_hip_state_update_args;

int strata_hip_state_update(const strata_hip_state_update_args* args, void* stream);

/* Library bookkeeping (no counterpart in the reference). */
const char* strata_hip_last_error(void);
/* ---------------------------------------------------------------------------
 * Pixel-stage block (no counterpart in this library's reference interface: the
 * block lives in physicsnemo, absent here; parameters adaln_bilinear_dw_{conv,proj}
 * per tests/regression_data/pixeldit_...param_order.txt:245-256, enabled by
 * use_bilinear_dw_gelu_project_adaln_pixel, screamcast/strata_wrappers.py:443,471-477).
 * This build's convention: the semantic tokens cond [B, Z, Yc, Xc, Cs] are upsampled
 * bilinearly by `factor` in y and x (align_corners = false), convolved depth-wise
 * with 3x3 taps (zero padding), biased and passed through GELU(tanh); a GEMM then
 * projects them to the six adaLN modulations of the pixel block, which uses
 * strata_hip_layer_norm_modulate and strata_hip_gated_add around its attention and MLP.
 * ------------------------------------------------------------------------- */
typedef struct strata_hip_upsample_dw_gelu_args {
  const void* cond;         /* [B, Z, Yc, Xc, Cs] bf16; strides (elements) over b, z, y, x; channels contiguous */
  void* out;                /* [B, Z, Yc*factor, Xc*factor, Cs] bf16; strides over b, z, y, x */
  const void* weight;       /* [9, Cs] bf16 taps, tap-major (tap 3 dy + dx of a Conv3d weight [Cs, 1, 1, 3, 3]) */
  const void* bias;         /* [Cs] bf16 or null */
  int32_t batch, depth, height, width, channels, factor;  /* height / width: the coarse grid */
  int64_t cond_stride[4];
  int64_t out_stride[4];
} strata_hip_upsample_dw_gelu_args;

int strata_hip_upsample_dw_gelu(const strata_hip_upsample_dw_gelu_args* args, void* stream);

/* out = LN(x) * (1 + scale) + shift per row (non-affine LayerNorm, fp32 statistics);
 * x, out, shift, scale: [M, C] bf16 with their own row strides (shift and scale may be
 * column slices of one modulation tensor). */
typedef struct strata_hip_layer_norm_modulate_args {
  const void* x;
  void* out;
  const void* shift;
  const void* scale;
  int64_t m, c;
  int64_t ldx, ldo, ld_shift, ld_scale;
  float eps;
  int32_t reserved;
} strata_hip_layer_norm_modulate_args;

int strata_hip_layer_norm_modulate(const strata_hip_layer_norm_modulate_args* args, void* stream);

/* out = res + gate * y elementwise ([M, C] bf16, each with its own row stride). */
typedef struct strata_hip_gated_add_args {
  const void* res;
  const void* gate;
  const void* y;
  void* out;
  int64_t m, c;
  int64_t ld_res, ld_gate, ld_y, ld_out;
} strata_hip_gated_add_args;

int strata_hip_gated_add(const strata_hip_gated_add_args* args, void* stream);

int strata_hip_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* STRATA_HIP_H */
