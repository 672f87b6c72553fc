// gfx950 (MI355X) kernels for the forward-Laplacian jet of the fixed 2 -> 64x4 -> 1 tanh MLP
// and its adjoint-jet backward, plus the C ABI declared in include/fused_hoad.h.
//
// Math (same as /root/reference/csrc/fused_residual.cu:16-23 and
// /root/reference/src/fused_hoad/backends/forward_laplacian.py:1-17): every point carries a
// jet (v, J0, J1, L) = (value, d/dx, d/dy, Laplacian) through the network.
//   linear:  z_v = W v + b,  z_J = W J,  z_L = W L
//   tanh:    a = tanh(z_v), s = 1 - a^2
//            v = a,  J = s z_J,  L = s z_L - 2 a s (z_J0^2 + z_J1^2)
//   output:  u = w_out . v + b_out,  lap = w_out . L
//
// Register layout. A wave owns a tile of 16 points. Each hidden layer is the product
// Z[64 x 64] = W[64 x 64] * H[64 x (4 components x 16 points)], done with
// v_mfma_f32_16x16x4f32 (FP32 in, FP32 accumulate). With m = lane % 16 and g = lane / 16, the
// MFMA accumulator of output block mb and component c holds, in register r,
//     Z[o = 16 mb + 4 g + r][c][point m].
// The contraction order is free, so k-step (ob, j) assigns lane group g the input neuron
// i = 16 ob + 4 g + j. Then the B operand a lane must supply at that step,
//     H[16 ob + 4 g + j][c][point m],
// is register j of the previous layer's accumulator (ob, c) in the same lane: a layer's output
// is already in the operand layout of the next layer, and the tanh-jet update (which needs the
// 4 components of one (neuron, point)) is local to a lane. Only the weights come from LDS.
//
// LDS weight layout. W[o][i] of a hidden layer is stored at 68 o - 3 (o & 3) + i (rows of 64
// with a per-row skew). The forward reads W[16 mb + m][16 ob + 4 g + j] (lane part
// 68 m - 3 (m & 3) + 4 g) and the backward's transposed product reads
// W[16 ob + 4 g + j][16 ib + m] (lane part 272 g + m). Both lane parts hit 64 distinct banks
// (mod 64) and the rest of each address is a compile-time immediate.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "fused_hoad.h"
#include "mlp_abi.h"

namespace fhoad {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kTile = 16;     // points per wave tile (the MFMA N dimension)
constexpr int kWRow = 68;     // skewed LDS row pitch, see the header comment
constexpr int kPlane = 4352;  // floats per skewed 64x64 plane (>= 68*63 - 9 + 64, multiple of 64)

// Small parameter blocks mirrored in LDS (float offsets inside s_small).
constexpr int kSmallW0 = 0;                                  // W0[64][2]
constexpr int kSmallB0 = kSmallW0 + kHidden * kInputs;        // b0[64]
constexpr int kSmallBh = kSmallB0 + kHidden;                  // b1..b3, [3][64]
constexpr int kSmallWout = kSmallBh + 3 * kHidden;            // w_out[64]
constexpr int kSmallBout = kSmallWout + kHidden;              // b_out
constexpr int kSmallFloats = kSmallBout + 4;

// Lane-dependent parts of the two LDS access patterns.
__device__ __forceinline__ int lane_rows(int m, int g) { return kWRow * m - 3 * (m & 3) + 4 * g; }
__device__ __forceinline__ int lane_cols(int m, int g) { return 272 * g + m; }

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 lds4(const float* p) { return *reinterpret_cast<const f4*>(p); }

// tanh and its derivative from t = exp(-2|z|), with r = 1 / (1 + t):
//   |tanh z| = (1 - t) r,   s = 1 - tanh^2 z = 4 t r^2.
// Written from the identity tanh z = (1 - e^{-2z}) / (1 + e^{-2z}) on v_exp_f32 / v_rcp_f32.
// s is formed without the 1 - a^2 cancellation, so it keeps full relative accuracy when tanh
// saturates; t flushes to 0 for |z| > ~44, giving a = +-1, s = 0.
__device__ __forceinline__ void tanh_and_slope(float z, float& a, float& s) {
  constexpr float kMinusTwoLog2e = -2.8853900817779268f;  // -2 / ln 2
  const float t = __builtin_amdgcn_exp2f(kMinusTwoLog2e * __builtin_fabsf(z));
  const float r = __builtin_amdgcn_rcpf(1.0f + t);
  a = __builtin_copysignf((1.0f - t) * r, z);
  s = (4.0f * t) * (r * r);
}

// Forward tanh jet: (z_v, z_J0, z_J1, z_L) -> (v, J0, J1, L).
__device__ __forceinline__ void tanh_jet(float zv, float zj0, float zj1, float zl, float& v,
                                         float& j0, float& j1, float& l) {
  float a, s;
  tanh_and_slope(zv, a, s);
  const float q = __builtin_fmaf(zj0, zj0, zj1 * zj1);
  v = a;
  j0 = s * zj0;
  j1 = s * zj1;
  l = __builtin_fmaf(-2.0f * a * s, q, s * zl);
}

// Adjoint of the tanh jet (/root/reference/csrc/fused_backward.cu:29-33), with s2 = -2 a s,
// s3 = 2 s (2 a^2 - s), q = z_J0^2 + z_J1^2:
//   zbar_v  = vbar s + (Jbar . z_J) s2 + Lbar (z_L s2 + q s3)
//   zbar_Jd = Jbar_d s + 2 Lbar s2 z_Jd
//   zbar_L  = Lbar s
// The adjoint (vbar, J0bar, J1bar, Lbar) is replaced by zbar in place.
__device__ __forceinline__ void tanh_jet_adjoint(float zv, float zj0, float zj1, float zl,
                                                 float& bv, float& bj0, float& bj1, float& bl) {
  float a, s;
  tanh_and_slope(zv, a, s);
  const float s2 = -2.0f * a * s;
  const float s3 = 2.0f * s * __builtin_fmaf(2.0f * a, a, -s);
  const float q = __builtin_fmaf(zj0, zj0, zj1 * zj1);
  const float dot = __builtin_fmaf(bj0, zj0, bj1 * zj1);
  const float curv = __builtin_fmaf(zl, s2, q * s3);
  const float lb2 = 2.0f * bl * s2;
  const float nv = __builtin_fmaf(bv, s, __builtin_fmaf(dot, s2, bl * curv));
  const float nj0 = __builtin_fmaf(bj0, s, lb2 * zj0);
  const float nj1 = __builtin_fmaf(bj1, s, lb2 * zj1);
  bv = nv;
  bj0 = nj0;
  bj1 = nj1;
  bl = bl * s;
}

// Copy the packed parameters into LDS: the three hidden W into skewed planes, the small
// blocks (W0, biases, w_out, b_out) verbatim. Reads are coalesced 4-byte loads, so the
// parameter buffer needs no particular alignment.
__device__ __forceinline__ void stage_parameters(const float* __restrict__ params, float* s_w,
                                                 float* s_small, int tid, int threads) {
  for (int k = tid; k < 3 * kHidden * kHidden; k += threads) {
    const int layer = k >> 12;
    const int o = (k >> 6) & 63;
    const int i = k & 63;
    s_w[layer * kPlane + kWRow * o - 3 * (o & 3) + i] =
        params[kHiddenBase + layer * kHiddenStride + (o << 6) + i];
  }
  for (int k = tid; k < kHidden * kInputs + kHidden; k += threads) {
    s_small[kSmallW0 + k] = params[k];  // W0 then b0 are contiguous in the ABI
  }
  for (int k = tid; k < 3 * kHidden; k += threads) {
    const int layer = k >> 6;
    s_small[kSmallBh + k] = params[kHiddenBase + layer * kHiddenStride + kHidden * kHidden + (k & 63)];
  }
  for (int k = tid; k < kHidden + 1; k += threads) {
    s_small[kSmallWout + k] = params[kOutputBase + k];
  }
}

// Layer-0 weights of the 4 neurons o = 16 mb + 4 g + r (r = 0..3) held by this lane.
struct Layer0Weights {
  f4 wx, wy, b;
};

__device__ __forceinline__ Layer0Weights layer0_weights(const float* s_small, int mb, int g) {
  const int o = 16 * mb + 4 * g;
  const f4 lo = lds4(s_small + kSmallW0 + 2 * o);
  const f4 hi = lds4(s_small + kSmallW0 + 2 * o + 4);
  Layer0Weights w;
  w.wx = f4{lo[0], lo[2], hi[0], hi[2]};
  w.wy = f4{lo[1], lo[3], hi[1], hi[3]};
  w.b = lds4(s_small + kSmallB0 + o);
  return w;
}

// Hidden-layer product acc[mb][c] += W[16 mb + ., :] H[:, c, .] with H in registers (see the
// header comment for the k-step assignment). w points at this lane's row base in the layer's
// LDS plane.
__device__ __forceinline__ void hidden_product(const float* w, const f4 (&h)[4][4],
                                               f4 (&acc)[4][4]) {
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) a[mb] = w[1088 * mb + 16 * ob + j];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[mb][c] = mfma(a[mb], h[ob][c][j], acc[mb][c]);
      }
    }
  }
}

// Transposed product hb[ib][c] = sum_o W[o][16 ib + .] zb[o][c][.]: the adjoint of a hidden
// layer's input. zb is in the same register layout as h; w points at this lane's column base.
__device__ __forceinline__ void hidden_product_t(const float* w, const f4 (&zb)[4][4],
                                                 f4 (&hb)[4][4]) {
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) {
#pragma unroll
    for (int c = 0; c < 4; ++c) hb[ib][c] = f4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) a[ib] = w[1088 * ob + 65 * j + 16 * ib];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
#pragma unroll
        for (int c = 0; c < 4; ++c) hb[ib][c] = mfma(a[ib], zb[ob][c][j], hb[ib][c]);
      }
    }
  }
}

__device__ __forceinline__ void bias_init(const float* s_small, int layer, int g, f4 (&acc)[4][4]) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    acc[mb][0] = lds4(s_small + kSmallBh + layer * kHidden + 16 * mb + 4 * g);
#pragma unroll
    for (int c = 1; c < 4; ++c) acc[mb][c] = f4{0.f, 0.f, 0.f, 0.f};
  }
}

__device__ __forceinline__ void apply_tanh_jet(const f4 (&z)[4][4], f4 (&h)[4][4]) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v, j0, j1, l;
      tanh_jet(z[mb][0][r], z[mb][1][r], z[mb][2][r], z[mb][3][r], v, j0, j1, l);
      h[mb][0][r] = v;
      h[mb][1][r] = j0;
      h[mb][2][r] = j1;
      h[mb][3][r] = l;
    }
  }
}

// Layer 0 in closed form: the input jet is (x, I, 0), so z_J = W0 columns and z_L = 0.
__device__ __forceinline__ void layer0_forward(const float* s_small, int g, float x0, float x1,
                                               f4 (&h)[4][4]) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const Layer0Weights w = layer0_weights(s_small, mb, g);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float zv = __builtin_fmaf(w.wx[r], x0, __builtin_fmaf(w.wy[r], x1, w.b[r]));
      float v, j0, j1, l;
      tanh_jet(zv, w.wx[r], w.wy[r], 0.0f, v, j0, j1, l);
      h[mb][0][r] = v;
      h[mb][1][r] = j0;
      h[mb][2][r] = j1;
      h[mb][3][r] = l;
    }
  }
}

__device__ __forceinline__ float sum_lane_groups(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// ---------------------------------------------------------------------------------------------
// Forward kernel (replaces fused_forward_laplacian_tiled_kernel<2>,
// /root/reference/csrc/fused_residual.cu:157-295). A grid of at most one workgroup per CU
// stages the weights once, then every wave walks 16-point tiles: tile t goes to workgroup
// t % grid, wave (t / grid) % kWaves, so small batches still spread over all CUs.
template <int kWaves>
__global__ void __launch_bounds__(kWaves * kWave)
forward_kernel(const float* __restrict__ coordinates, const float* __restrict__ params,
               float* __restrict__ output, float* __restrict__ laplacian, int64_t batch,
               int64_t tiles) {
  __shared__ __attribute__((aligned(16))) float s_w[3 * kPlane];
  __shared__ __attribute__((aligned(16))) float s_small[kSmallFloats];
  stage_parameters(params, s_w, s_small, threadIdx.x, kWaves * kWave);
  __syncthreads();

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int m = lane & 15;
  const int g = lane >> 4;
  const float* w_lane = s_w + lane_rows(m, g);
  const int64_t step = static_cast<int64_t>(gridDim.x) * kWaves;

  for (int64_t tile = blockIdx.x + static_cast<int64_t>(wave) * gridDim.x; tile < tiles;
       tile += step) {
    const int64_t point = tile * kTile + m;
    const bool active = point < batch;
    float x0 = 0.0f, x1 = 0.0f;
    if (active) {
      x0 = coordinates[2 * point];
      x1 = coordinates[2 * point + 1];
    }
    f4 h[4][4];
    layer0_forward(s_small, g, x0, x1, h);
    for (int layer = 0; layer < 3; ++layer) {
      f4 acc[4][4];
      bias_init(s_small, layer, g, acc);
      hidden_product(w_lane + layer * kPlane, h, acc);
      apply_tanh_jet(acc, h);
    }
    float u = 0.0f, lap = 0.0f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const f4 w = lds4(s_small + kSmallWout + 16 * mb + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        u = __builtin_fmaf(w[r], h[mb][0][r], u);
        lap = __builtin_fmaf(w[r], h[mb][3][r], lap);
      }
    }
    u = sum_lane_groups(u);
    lap = sum_lane_groups(lap);
    if (g == 0 && active) {
      output[point] = u + s_small[kSmallBout];
      laplacian[point] = lap;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Backward (replaces fused_backward_occupancy_kernel<false,true,false,true> and the host-side
// partials.sum(0), /root/reference/csrc/fused_backward.cu:424-850, 859-934).
//
// One workgroup per CU, 4 waves (one per SIMD, up to 512 registers each), 64-point workgroup
// tiles (16 points per wave). Per tile:
//   1. every wave re-runs the forward for its 16 points, keeping the pre-activations z in
//      registers;
//   2. the adjoint is seeded from the linear output layer and walked back through layers 3..1:
//      tanh-jet adjoint in registers, dW += zbar h_prev^T, hbar = W^T zbar (registers), and
//      finally layer 0 in closed form;
//   3. dW contracts over the points of all 4 waves: zbar and h_prev are staged in LDS (two
//      components at a time) and wave w owns output rows 16 w .. 16 w + 15 of every dW.
//      Bias, W0 and w_out gradients are reduced over points by the same owner waves.
// Weight gradients accumulate in registers across the tiles of a "slot": slot s takes the
// workgroup tiles s, s + slots, s + 2 slots, ... in that order and writes one partial row.
// A second kernel sums the rows in a fixed tree. The slot count depends only on the batch,
// so the result does not depend on the grid size. No float atomics anywhere.
constexpr int kBwdWaves = 4;
constexpr int kBwdTile = kBwdWaves * kTile;  // 64 points
constexpr int kMaxSlots = 256;
constexpr int kRowStride = 12800;            // floats per partial row (>= 12737)
constexpr int kReduceGroups = 16;            // fixed reduction tree: 16 groups of 16 slots
static_assert(kMaxSlots % kReduceGroups == 0, "reduction tree must tile the slots");

__device__ __forceinline__ f4 zero4() { return f4{0.f, 0.f, 0.f, 0.f}; }

// Stage two jet components of this wave's zbar and h_prev into the dW staging buffer. Rows
// are the workgroup tile's 64 points, columns the 64 neurons, same skewed pitch as weights.
// zb components (c0, c0+1) go to planes 0, 1 and h_prev components to planes 2, 3.
__device__ __forceinline__ void stage_write(float* stage_lane, int mb, int r, float z_a,
                                            float z_b, float h_a, float h_b) {
  float* p = stage_lane + 16 * mb + r;
  p[0] = z_a;
  p[kPlane] = z_b;
  p[2 * kPlane] = h_a;
  p[3 * kPlane] = h_b;
}

// dW[16 w + ., 16 nb + .] += sum over (2 staged components, 64 points) of zbar h_prev^T.
// Lane (m, g) reads zbar[16 w + m][p] and h_prev[16 nb + m][p] for p = 16 s + 4 g + k, so the
// MFMA contracts over points. Returns the sum of this lane's plane-0 zbar reads (the bias
// gradient partial when plane 0 holds zbar_v).
__device__ __forceinline__ float dw_product(const float* stage_cols, int w, f4 (&dw)[4]) {
  float bias = 0.0f;
#pragma unroll
  for (int cc = 0; cc < 2; ++cc) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int off = cc * kPlane + 1088 * s + 65 * k;
        const float a = stage_cols[off + 16 * w];
        if (cc == 0) bias += a;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          dw[nb] = mfma(a, stage_cols[off + 2 * kPlane + 16 * nb], dw[nb]);
        }
      }
    }
  }
  return bias;
}

// Sum of staged plane `plane` over the 64 points for neuron 16 w + m, complete in every lane.
__device__ __forceinline__ float plane_sum(const float* stage_cols, int plane, int w) {
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
#pragma unroll
    for (int k = 0; k < 4; ++k) acc += stage_cols[plane * kPlane + 1088 * s + 65 * k + 16 * w];
  }
  return sum_lane_groups(acc);
}

// Replace a hidden layer's pre-activation z by its adjoint zbar, given the adjoint hb of the
// layer's output (tanh-jet adjoint, lane-local).
__device__ __forceinline__ void tanh_adjoint_in_place(f4 (&z)[4][4], const f4 (&hb)[4][4]) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float bv = hb[mb][0][r], bj0 = hb[mb][1][r], bj1 = hb[mb][2][r], bl = hb[mb][3][r];
      tanh_jet_adjoint(z[mb][0][r], z[mb][1][r], z[mb][2][r], z[mb][3][r], bv, bj0, bj1, bl);
      z[mb][0][r] = bv;
      z[mb][1][r] = bj0;
      z[mb][2][r] = bj1;
      z[mb][3][r] = bl;
    }
  }
}

// dW += zbar h_prev^T over the workgroup tile, in two passes of two jet components, where
// h_prev = tanh_jet(zp) is rebuilt from the previous layer's pre-activation (or, with
// kFromLayer0, from layer 0's closed form z = (W0 x + b0, W0[:,0], W0[:,1], 0)). Adds the
// bias gradient sum_p zbar_v to g_bias.
template <bool kFromLayer0>
__device__ __forceinline__ void stage_and_dw(const f4 (&zbar)[4][4], const f4 (&zp)[4][4],
                                             f4 (&dw)[4], float& g_bias, float* stage_lane,
                                             const float* stage_cols, const float* s_small,
                                             int w, int g, float x0, float x1) {
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    __syncthreads();  // previous readers of the staging buffer are done
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      Layer0Weights w0;
      if (kFromLayer0) w0 = layer0_weights(s_small, mb, g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float pv, pj0, pj1, pl;
        if (kFromLayer0) {
          pv = __builtin_fmaf(w0.wx[r], x0, __builtin_fmaf(w0.wy[r], x1, w0.b[r]));
          pj0 = w0.wx[r];
          pj1 = w0.wy[r];
          pl = 0.0f;
        } else {
          pv = zp[mb][0][r];
          pj0 = zp[mb][1][r];
          pj1 = zp[mb][2][r];
          pl = zp[mb][3][r];
        }
        float hv, hj0, hj1, hl;
        tanh_jet(pv, pj0, pj1, pl, hv, hj0, hj1, hl);
        if (half == 0) {
          stage_write(stage_lane, mb, r, zbar[mb][0][r], zbar[mb][1][r], hv, hj0);
        } else {
          stage_write(stage_lane, mb, r, zbar[mb][2][r], zbar[mb][3][r], hj1, hl);
        }
      }
    }
    __syncthreads();
    const float bias = dw_product(stage_cols, w, dw);
    if (half == 0) g_bias += sum_lane_groups(bias);
  }
}

// Only z of hidden layers 2 and 3 is kept from the forward recompute; z of hidden layer 1 is
// recomputed from x just before it is needed. That keeps the live state near 240 registers
// per lane, so nothing spills.
__global__ void __launch_bounds__(kBwdWaves * kWave, 1)
backward_kernel(const float* __restrict__ coordinates, const float* __restrict__ params,
                const float* __restrict__ grad_output, const float* __restrict__ grad_laplacian,
                float* __restrict__ grad_coordinates, float* __restrict__ partials,
                int64_t batch, int64_t tiles, int slots) {
  __shared__ __attribute__((aligned(16))) float s_w[3 * kPlane];
  __shared__ __attribute__((aligned(16))) float s_small[kSmallFloats];
  __shared__ __attribute__((aligned(16))) float s_stage[4 * kPlane];
  __shared__ float s_red[kBwdWaves];
  stage_parameters(params, s_w, s_small, threadIdx.x, kBwdWaves * kWave);
  __syncthreads();

  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int m = lane & 15;
  const int g = lane >> 4;
  const float* w_rows = s_w + lane_rows(m, g);
  const float* w_cols = s_w + lane_cols(m, g);
  float* stage_lane = s_stage + 1088 * w + lane_rows(m, g);
  const float* stage_cols = s_stage + lane_cols(m, g);

  for (int slot = blockIdx.x; slot < slots; slot += gridDim.x) {
    f4 dw[3][4];
#pragma unroll
    for (int l = 0; l < 3; ++l) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) dw[l][nb] = zero4();
    }
    float g_bh[3] = {0.f, 0.f, 0.f};
    float g_w0x = 0.f, g_w0y = 0.f, g_b0 = 0.f, g_wout = 0.f, g_bout = 0.f;

    for (int64_t tile = slot; tile < tiles; tile += slots) {
      const int64_t point = tile * kBwdTile + kTile * w + m;
      const bool active = point < batch;
      float x0 = 0.f, x1 = 0.f, gu = 0.f, gl = 0.f;
      if (active) {
        x0 = coordinates[2 * point];
        x1 = coordinates[2 * point + 1];
        gu = grad_output[point];
        gl = grad_laplacian[point];
      }

      // ---- 1. forward recompute ----
      f4 h[4][4];
      f4 z2[4][4], z3[4][4];
      layer0_forward(s_small, g, x0, x1, h);
      {
        f4 z1[4][4];
        bias_init(s_small, 0, g, z1);
        hidden_product(w_rows, h, z1);
        apply_tanh_jet(z1, h);
      }
      bias_init(s_small, 1, g, z2);
      hidden_product(w_rows + kPlane, h, z2);
      apply_tanh_jet(z2, h);
      bias_init(s_small, 2, g, z3);
      hidden_product(w_rows + 2 * kPlane, h, z3);
      apply_tanh_jet(z3, h);

      // ---- 2. output layer: w_out / b_out gradients and the adjoint seed ----
      __syncthreads();  // the staging buffer is free
      f4 hb[4][4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const f4 wo = lds4(s_small + kSmallWout + 16 * mb + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          stage_lane[16 * mb + r] = __builtin_fmaf(gu, h[mb][0][r], gl * h[mb][3][r]);
          hb[mb][0][r] = gu * wo[r];
          hb[mb][1][r] = 0.0f;
          hb[mb][2][r] = 0.0f;
          hb[mb][3][r] = gl * wo[r];
        }
      }
      {
        float su = gu;
        su += __shfl_xor(su, 1);
        su += __shfl_xor(su, 2);
        su += __shfl_xor(su, 4);
        su += __shfl_xor(su, 8);
        if (lane == 0) s_red[w] = su;
      }
      __syncthreads();
      g_wout += plane_sum(stage_cols, 0, w);
      g_bout += ((s_red[0] + s_red[1]) + s_red[2]) + s_red[3];

      // ---- 3. hidden layer 3 ----
      tanh_adjoint_in_place(z3, hb);
      stage_and_dw<false>(z3, z2, dw[2], g_bh[2], stage_lane, stage_cols, s_small, w, g, x0, x1);
      hidden_product_t(w_cols + 2 * kPlane, z3, hb);

      // ---- 4. hidden layer 2 (needs hidden layer 1's z: recompute it) ----
      tanh_adjoint_in_place(z2, hb);
      f4 z1[4][4];
      layer0_forward(s_small, g, x0, x1, h);
      bias_init(s_small, 0, g, z1);
      hidden_product(w_rows, h, z1);
      stage_and_dw<false>(z2, z1, dw[1], g_bh[1], stage_lane, stage_cols, s_small, w, g, x0, x1);
      hidden_product_t(w_cols + kPlane, z2, hb);

      // ---- 5. hidden layer 1 ----
      tanh_adjoint_in_place(z1, hb);
      stage_and_dw<true>(z1, z1, dw[0], g_bh[0], stage_lane, stage_cols, s_small, w, g, x0, x1);
      hidden_product_t(w_cols, z1, hb);

      // ---- 6. layer 0 in closed form ----
      float gx0 = 0.f, gx1 = 0.f;
      __syncthreads();  // staging buffer free again
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const Layer0Weights w0 = layer0_weights(s_small, mb, g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float zv = __builtin_fmaf(w0.wx[r], x0, __builtin_fmaf(w0.wy[r], x1, w0.b[r]));
          float bv = hb[mb][0][r], bj0 = hb[mb][1][r], bj1 = hb[mb][2][r], bl = hb[mb][3][r];
          tanh_jet_adjoint(zv, w0.wx[r], w0.wy[r], 0.0f, bv, bj0, bj1, bl);
          gx0 = __builtin_fmaf(w0.wx[r], bv, gx0);
          gx1 = __builtin_fmaf(w0.wy[r], bv, gx1);
          float* p = stage_lane + 16 * mb + r;
          p[0] = __builtin_fmaf(bv, x0, bj0);       // dW0[o][0] contribution
          p[kPlane] = __builtin_fmaf(bv, x1, bj1);  // dW0[o][1]
          p[2 * kPlane] = bv;                       // db0[o]
        }
      }
      gx0 = sum_lane_groups(gx0);
      gx1 = sum_lane_groups(gx1);
      if (g == 0 && active) {
        grad_coordinates[2 * point] = gx0;
        grad_coordinates[2 * point + 1] = gx1;
      }
      __syncthreads();
      g_w0x += plane_sum(stage_cols, 0, w);
      g_w0y += plane_sum(stage_cols, 1, w);
      g_b0 += plane_sum(stage_cols, 2, w);
    }

    // ---- this slot's partial row: every entry written by exactly one lane ----
    float* row = partials + static_cast<int64_t>(slot) * kRowStride;
#pragma unroll
    for (int l = 0; l < 3; ++l) {
      float* wrow = row + kHiddenBase + l * kHiddenStride;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) wrow[(16 * w + 4 * g + r) * kHidden + 16 * nb + m] = dw[l][nb][r];
      }
      if (g == 0) wrow[kHidden * kHidden + 16 * w + m] = g_bh[l];
    }
    if (g == 0) {
      const int o = 16 * w + m;
      row[kInputs * o] = g_w0x;
      row[kInputs * o + 1] = g_w0y;
      row[kLayer0Bias + o] = g_b0;
      row[kOutputBase + o] = g_wout;
    }
    if (threadIdx.x == 0) row[kOutputBase + kHidden] = g_bout;
    __syncthreads();  // s_red and the staging buffer are reused by the next slot
  }
}

// grad[k] = sum over slots of partials[slot][k], in a fixed tree: 16 groups of 16 consecutive
// slots are summed in slot order, then the 16 group sums in group order. Slots at or beyond
// `slots` are skipped (they would add +0.0f).
__global__ void __launch_bounds__(kReduceGroups * 64)
reduce_partials_kernel(const float* __restrict__ partials, int slots, float* __restrict__ grad) {
  __shared__ float s_part[kReduceGroups][64];
  const int col = threadIdx.x & 63;
  const int group = threadIdx.x >> 6;
  const int k = blockIdx.x * 64 + col;
  constexpr int kPerGroup = kMaxSlots / kReduceGroups;
  float acc = 0.0f;
  if (k < kParameterCount) {
    float v[kPerGroup];
#pragma unroll
    for (int i = 0; i < kPerGroup; ++i) {
      const int slot = group * kPerGroup + i;
      v[i] = slot < slots ? partials[static_cast<int64_t>(slot) * kRowStride + k] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kPerGroup; ++i) acc += v[i];
  }
  s_part[group][col] = acc;
  __syncthreads();
  if (group == 0 && k < kParameterCount) {
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < kReduceGroups; ++i) total += s_part[i][col];
    grad[k] = total;
  }
}

__global__ void fill_zero_kernel(float* __restrict__ out, int64_t n) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (k < n) out[k] = 0.0f;
}

// ---------------------------------------------------------------------------------------------
// Host side.

constexpr int kFwdWaves = 8;

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
  va_end(args);
  return status;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(FHOAD_ERROR_DEVICE, "%s launch failed: %s", what, hipGetErrorString(err));
  }
  return FHOAD_SUCCESS;
}

// Compute units of the current device, queried once per device.
int current_device_cus(int* cus) {
  constexpr int kMaxDevices = 64;
  static int cached[kMaxDevices] = {};
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(FHOAD_ERROR_DEVICE, "hipGetDevice: %s", hipGetErrorString(err));
  if (device >= 0 && device < kMaxDevices && cached[device] > 0) {
    *cus = cached[device];
    return FHOAD_SUCCESS;
  }
  int count = 0;
  err = hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device);
  if (err != hipSuccess) {
    return fail(FHOAD_ERROR_DEVICE, "hipDeviceGetAttribute: %s", hipGetErrorString(err));
  }
  if (count < 1) count = 1;
  if (device >= 0 && device < kMaxDevices) cached[device] = count;
  *cus = count;
  return FHOAD_SUCCESS;
}

int64_t backward_tiles(int64_t batch) { return (batch + kBwdTile - 1) / kBwdTile; }

int backward_slots(int64_t batch) {
  return static_cast<int>(std::min<int64_t>(backward_tiles(batch), kMaxSlots));
}

}  // namespace
}  // namespace fhoad

using namespace fhoad;

extern "C" int fhoad_abi_version(void) { return FHOAD_ABI_VERSION; }

extern "C" int64_t fhoad_parameter_count(void) { return kParameterCount; }

extern "C" const char* fhoad_status_string(int status) {
  switch (status) {
    case FHOAD_SUCCESS: return "success";
    case FHOAD_ERROR_INVALID_VERSION: return "invalid version";
    case FHOAD_ERROR_INVALID_VALUE: return "invalid value";
    case FHOAD_ERROR_MISALIGNED: return "misaligned pointer";
    case FHOAD_ERROR_WORKSPACE: return "workspace too small";
    case FHOAD_ERROR_DEVICE: return "device error";
    default: return "unknown status";
  }
}

extern "C" const char* fhoad_last_error(void) { return g_last_error; }

extern "C" int fhoad_forward_laplacian(const float* coordinates, const float* parameters,
                                       float* output, float* laplacian, int64_t batch,
                                       int version, void* stream) {
  if (version < 0 || version > 5) return fail(FHOAD_ERROR_INVALID_VERSION, "version must be 0 to 5");
  if (batch < 0) return fail(FHOAD_ERROR_INVALID_VALUE, "batch must be non-negative");
  if (batch == 0) return FHOAD_SUCCESS;
  if (!coordinates || !parameters || !output || !laplacian) {
    return fail(FHOAD_ERROR_INVALID_VALUE, "null device pointer");
  }
  int cus = 0;
  if (int st = current_device_cus(&cus)) return st;
  const int64_t tiles = (batch + kTile - 1) / kTile;
  const int grid = static_cast<int>(std::min<int64_t>(tiles, cus));
  hipLaunchKernelGGL(forward_kernel<kFwdWaves>, dim3(grid), dim3(kFwdWaves * kWave), 0,
                     static_cast<hipStream_t>(stream), coordinates, parameters, output, laplacian,
                     batch, tiles);
  return check_launch("forward_kernel");
}

extern "C" size_t fhoad_backward_workspace_size(int64_t batch) {
  if (batch <= 0) return 0;
  return static_cast<size_t>(backward_slots(batch)) * kRowStride * sizeof(float);
}

extern "C" int fhoad_forward_laplacian_backward(const float* coordinates, const float* parameters,
                                                const float* grad_output,
                                                const float* grad_laplacian,
                                                float* grad_parameters, float* grad_coordinates,
                                                void* workspace, size_t workspace_bytes,
                                                int64_t batch, int version, void* stream) {
  if (version < 1 || version > 6) {
    return fail(FHOAD_ERROR_INVALID_VERSION, "backward version must be 1 to 6");
  }
  if (batch < 0) return fail(FHOAD_ERROR_INVALID_VALUE, "batch must be non-negative");
  if (!parameters || !grad_parameters) return fail(FHOAD_ERROR_INVALID_VALUE, "null device pointer");
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  if (batch == 0) {
    hipLaunchKernelGGL(fill_zero_kernel, dim3((kParameterCount + 255) / 256), dim3(256), 0, hs,
                       grad_parameters, static_cast<int64_t>(kParameterCount));
    return check_launch("fill_zero_kernel");
  }
  if (!coordinates || !grad_output || !grad_laplacian || !grad_coordinates) {
    return fail(FHOAD_ERROR_INVALID_VALUE, "null device pointer");
  }
  const size_t needed = fhoad_backward_workspace_size(batch);
  if (!workspace || workspace_bytes < needed) {
    return fail(FHOAD_ERROR_WORKSPACE, "workspace holds %zu bytes, %zu needed", workspace_bytes,
                needed);
  }
  int cus = 0;
  if (int st = current_device_cus(&cus)) return st;
  const int64_t tiles = backward_tiles(batch);
  const int slots = backward_slots(batch);
  int grid = std::min(slots, cus);
  // FUSED_HOAD_BWD_BLOCKS caps the persistent grid, as in the reference
  // (fused_backward.cu:873-880). Here it changes only which workgroup computes a slot, never
  // the arithmetic, so gradients stay bitwise identical.
  if (const char* env = std::getenv("FUSED_HOAD_BWD_BLOCKS")) {
    const long cap = std::atol(env);
    if (cap > 0) grid = static_cast<int>(std::min<long>(grid, cap));
  }
  float* partials = static_cast<float*>(workspace);
  hipLaunchKernelGGL(backward_kernel, dim3(grid), dim3(kBwdWaves * kWave), 0, hs, coordinates,
                     parameters, grad_output, grad_laplacian, grad_coordinates, partials, batch,
                     tiles, slots);
  if (int st = check_launch("backward_kernel")) return st;
  hipLaunchKernelGGL(reduce_partials_kernel, dim3((kParameterCount + 63) / 64),
                     dim3(kReduceGroups * 64), 0, hs, partials, slots, grad_parameters);
  return check_launch("reduce_partials_kernel");
}
