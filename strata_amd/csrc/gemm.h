// GEMM parameters of the hand-written kernels (gemm.hip).
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

}  // namespace strata
