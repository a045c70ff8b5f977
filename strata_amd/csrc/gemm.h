// GEMM parameters shared by the hand-written kernels (gemm.hip) and the
// hipBLASLt path for plain GEMMs (gemm_lt.cpp).
#pragma once

#include "common.h"

namespace strata {

struct GemmParams {
  const bf16* x;
  const bf16* w;
  const bf16* bias;
  const bf16* res;
  bf16* out;
  bf16* out2;  // the SAVE instance of the DMA kernel: gelu'(pre-activation), row stride ldo
  int64_t M, N, K;
  int64_t ldx, ldw, ldr, ldo;
  int act;
  int res_op;  // strata_hip_res_op: the residual is added or multiplied
  int mt, nt;  // tiles along M and N
};

// gemm_lt's answer when it does not take a GEMM (fused activation, multiplied
// residual, no hipBLASLt algorithm, or STRATA_HIP_GEMM=native): the caller
// runs the hand-written kernel instead.
constexpr int GEMM_LT_DECLINED = 1;
// gemm_lt's answer when hipBLASLt cannot create its handle on this device:
// the call fails (reported through strata_hip_last_error), nothing is latched.
constexpr int GEMM_LT_FAILED = 2;

// False when the environment sets STRATA_HIP_GEMM=native (every GEMM on the
// hand-written kernels, e.g. to compare the two paths).
bool gemm_lt_enabled();

// out = x @ w^T (+ bias) (+ residual) through hipBLASLt; STRATA_HIP_OK,
// GEMM_LT_DECLINED or GEMM_LT_FAILED.
int gemm_lt(const GemmParams& p, hipStream_t stream);

}  // namespace strata
