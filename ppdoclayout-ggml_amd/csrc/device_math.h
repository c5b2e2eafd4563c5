// Device-side helpers shared by the kernels: the activation codes of the GEMM
// / elementwise epilogues, the box-refinement inverse sigmoid and the
// XCD-aware block order.
#pragma once
#include <hip/hip_runtime.h>

#include "ppdl_internal.h"

namespace ppdl {

// GELU (erf form) and sigmoid, kept out of line: the epilogues apply the
// activation to many unrolled values, and the erf code inlined at each of
// them multiplies the code a kernel fetches.
__device__ __noinline__ float act_rare(float v, int act) {
    if (act == kActGelu) return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
    return 1.0f / (1.0f + expf(-v));
}

// 0 none, 1 ReLU, 2 SiLU, 3 GELU (erf form), 4 sigmoid: ggml's relu / silu /
// gelu_erf / sigmoid
__device__ __forceinline__ float act_f(float v, int act) {
    if (act == kActRelu) return v > 0.0f ? v : 0.0f;
    if (act == kActSilu) return v / (1.0f + expf(-v));
    if (act == kActGelu || act == kActSigmoid) return act_rare(v, act);
    return v;
}

// act_f with the activation fixed at compile time (A < 0: the runtime code
// act): the same formulas, without the other activations' code in kernels
// that apply it to many unrolled values.
template <int A>
__device__ __forceinline__ float act_t(float v, int act) {
    if constexpr (A < 0) return act_f(v, act);
    else return act_f(v, A);
}

// src/ppdoclayout.cpp:589-594: clamp to [0,1], log(max(x,1e-5)) - log(max(1-x,1e-5))
__device__ __forceinline__ float inv_sigmoid(float x) {
    x = fminf(fmaxf(x, 0.0f), 1.0f);
    const float x1 = fminf(fmaxf(x, 1e-5f), 1.0f);
    const float x2 = fminf(fmaxf(1.0f - x, 1e-5f), 1.0f);
    return logf(x1) - logf(x2);
}

// Blocks are dispatched round-robin over the 8 XCDs (hardware id % 8).  The
// logical block of hardware block `hw` out of `n`: each XCD gets a contiguous
// range of logical blocks, so blocks sharing operands hit the same L2.
__device__ __forceinline__ int xcd_remap(int hw, int n) {
    const int q = n >> 3, r = n & 7;
    const int xcd = hw & 7, slot = hw >> 3;
    return xcd * q + (xcd < r ? xcd : r) + slot;
}

// Sum over the 64 lanes of a wave, the same value in every lane: DPP steps
// inside each row of 16 lanes (quad swaps, then half-row and row mirrors),
// then the four row totals read out and added in lane order.  Every step
// pairs equal partial sums, so all lanes hold bit-identical results.
__device__ __forceinline__ float wave_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));   // [1,0,3,2]
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));   // [2,3,0,1]
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));  // half mirror
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));  // row mirror
    const int xi = __float_as_int(x);
    return ((__int_as_float(__builtin_amdgcn_readlane(xi, 0)) + __int_as_float(__builtin_amdgcn_readlane(xi, 16))) +
            __int_as_float(__builtin_amdgcn_readlane(xi, 32))) +
           __int_as_float(__builtin_amdgcn_readlane(xi, 48));
}

// box refinement (src/ppdoclayout.cpp:860-862): sigmoid(delta + inv_sigmoid(ref))
// Out of line for the same reason as act_rare: only the box-head GEMM's
// epilogue takes it, and every epilogue would otherwise carry its code.
__device__ __noinline__ float refine_box(float delta, float ref) {
    return 1.0f / (1.0f + expf(-(delta + inv_sigmoid(ref))));
}

}  // namespace ppdl
