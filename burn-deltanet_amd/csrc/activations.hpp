// The front-end's elementwise functions, shared by dn_frontend and
// dn_block_step so that both evaluate them identically.
#pragma once

#include "dn_common.hpp"

namespace dn {

// σ(x) = 1 / (1 + e^−x) with the hardware reciprocal (1 ulp).
__device__ inline float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// QkActivation / ConvActivation (norm.rs:38-51, conv.rs:39-44).
__device__ inline float activate(float x, int kind) {
  switch (kind) {
    case DN_ACT_SILU: return x * sigmoidf_(x);
    case DN_ACT_RELU: return fmaxf(x, 0.f);
    case DN_ACT_ELU_PLUS_ONE: return x < 0.f ? __expf(x) : x + 1.0f;
    default: return x;
  }
}

}  // namespace dn
