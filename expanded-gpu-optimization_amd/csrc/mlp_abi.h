// Shape and packed-parameter layout of the fixed 2 -> 64x4 -> 1 tanh MLP.
//
// Same offsets as /root/reference/csrc/mlp_abi.cuh:8-17 and
// /root/reference/src/fused_hoad/parameters.py:28-48, so a buffer packed for the reference
// kernels is valid here unchanged.
#pragma once

namespace fhoad {

constexpr int kInputs = 2;
constexpr int kHidden = 64;
constexpr int kHiddenLayers = 4;  // layer 0 (2 -> 64) plus three 64 -> 64 layers

constexpr int kLayer0Bias = kHidden * kInputs;                            // 128
constexpr int kHiddenBase = kLayer0Bias + kHidden;                        // 192
constexpr int kHiddenStride = kHidden * kHidden + kHidden;                // 4160
constexpr int kOutputBase = kHiddenBase + (kHiddenLayers - 1) * kHiddenStride;  // 12672
constexpr int kParameterCount = kOutputBase + kHidden + 1;               // 12737
static_assert(kParameterCount == 12737, "parameter ABI drifted from parameters.py");
static_assert(kHiddenBase % 4 == 0 && kHiddenStride % 4 == 0, "hidden blocks are float4-aligned");

}  // namespace fhoad
