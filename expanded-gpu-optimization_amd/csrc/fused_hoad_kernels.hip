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
// Scaled jet. With c = -2 log2(e) and lambda = log2(e), kernels carry the layer outputs as
//   (v', J0', J1', L') = (c v / 4, J0 / 2, J1 / 2, lambda L / 4)
// and stage the hidden weights as 4 W and the value biases as c b (exact power-of-two factors
// aside from c). The pre-activations then come out of the MFMAs as
//   z'_v = 4 W (c v / 4) + c b = c z_v,   z'_J = 4 W (J / 2) = 2 z_J,   z'_L = lambda z_L,
// and with s' = s / 4 and q' = |z'_J|^2 = 4 q the tanh jet keeps its form:
//   v' = (c / 4) tanh z_v,   J' = s' z'_J,   L' = s' (z'_L + v' q') = lambda L / 4
// (because c = -2 lambda), with the same scales at every layer. exp(-2 z_v) is exp2(z'_v) with
// no multiply, and (v', s') take 3 VALU + 2 transcendental instructions (tanh_scaled). Layer 0
// uses z'_J = 2 W0 columns; w_out is staged as 4 w_out / c and 4 w_out / lambda for u and lap.
// The backward is backpropagation through this scaled network (weights 4 W): its dW sums are
// of d/d(4 W), so the partial rows take a factor 4; bias gradients take c; layer-0 weight
// gradients c for the x terms and 2 for the z_J terms. FP32 MFMA runs on the same SIMD issue
// slots as VALU work on gfx950 (measured: they do not co-execute), so every VALU instruction
// saved in the jet update is MFMA time recovered.
//
// LDS weight layouts. The forward kernel keeps W in MFMA operand order (one 16-byte read per
// k-step, see stage_operand_weights); its small-batch form (forward_split_kernel) keeps only a
// wave's 16 rows, in registers. The backward kernels (backward_kernel, and
// backward_split_kernel for small batches) need both W and W^T operands from one copy:
// W[o][i] at 68 o + i, read as W[16 mb + m][16 ob + 4 g + j], j = 0..3 (16 bytes) for the forward
// recompute and as W[16 ob + 4 g + j][16 ib + m] (4 bytes) for W^T zbar.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
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
constexpr int kWRow = 68;     // LDS row pitch of the backward's 64-wide rows
constexpr int kPlane = 4352;  // floats per 64 x 68 LDS plane

// Scale factors of the carried jet (see the header comment).
constexpr float kC = -2.8853900817779268f;       // c = -2 log2(e)
constexpr float kLambda = 1.4426950408889634f;   // lambda = log2(e)
constexpr float kKappa = -0.96090602783640284f;  // -8 / c^2 (tanh_jet_adjoint_vs)
constexpr float kHalfC = 0.5f * kC;              // c / 2 (layer-0 weight gradients)

// Small parameter blocks in LDS (float offsets inside s_small), each [64] over neurons.
constexpr int kSmallCwx = 0;                       // c W0[:, 0]
constexpr int kSmallCwy = kSmallCwx + kHidden;     // c W0[:, 1]
constexpr int kSmallCb0 = kSmallCwy + kHidden;     // c b0
constexpr int kSmallWx = kSmallCb0 + kHidden;      // 2 W0[:, 0] (layer 0's z'_J0)
constexpr int kSmallWy = kSmallWx + kHidden;       // 2 W0[:, 1]
constexpr int kSmallQ0 = kSmallWy + kHidden;       // 4 (W0[:, 0]^2 + W0[:, 1]^2) = |z'_J|^2
constexpr int kSmallBh = kSmallQ0 + kHidden;       // c b1..b3, [3][64]
constexpr int kSmallWoutV = kSmallBh + 3 * kHidden;  // 4 w_out / c
constexpr int kSmallWoutL = kSmallWoutV + kHidden;   // 4 w_out / lambda
constexpr int kSmallBout = kSmallWoutL + kHidden;    // b_out
constexpr int kSmallFloats = kSmallBout + 4;

// Lane-dependent parts of the backward's two LDS access patterns on pitch-68 planes (value
// (row, col) at 68 row + col): reading 4 consecutive columns of row m (16 bytes at
// 68 m + 4 g) and reading one column m of rows 4 g + j (4 bytes at 272 g + m + 68 j). In both,
// the 64 lanes cover distinct banks per 16-lane group, and the remaining offsets are immediates.
__device__ __forceinline__ int lane_rows(int m, int g) { return kWRow * m + 4 * g; }
__device__ __forceinline__ int lane_cols(int m, int g) { return 272 * g + m; }

// The backward's dW staging buffer: six planes of [neuron row R][tile point p] in the weight
// planes' layout, (R, p) at 68 R + p. Planes 0..2 hold zbar of the three "early" jet
// components (early_component(e) in plane e), planes 3..5 h_prev of the same components; the
// "late" component (J1) goes into planes 0 and 3 once the products of plane pair (0, 3) are done.
// They are written 4 bytes per lane (lane (m, g) of wave w: rows 4 g + r of a 16-row block, point
// 16 w + m; base lane_cols(m, g) + 16 w, conflict-free) and read 16 bytes per lane (row m,
// points 4 g .. 4 g + 3 of a 16-point block; base lane_rows(m, g); 4 bank-conflict cycles per
// read on gfx950, which overlap the MFMAs that consume them). Six planes at pitch 68 (104 KB)
// fit beside the 52 KB of weight planes; at the conflict-free pitch 80 only four would.
constexpr int kStagePlanes = 6;
__device__ __forceinline__ constexpr int early_component(int e) { return e == 0 ? 0 : e == 1 ? 3 : 1; }
constexpr int kLateComponent = 2;

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 lds4(const float* p) { return *reinterpret_cast<const f4*>(p); }

// tanh in the scaled jet, four values at a time. Input zv = c z_v; outputs v = (c / 4) tanh(z_v)
// and s = (1 - tanh^2 z_v) / 4. With t = exp(-2 z_v) = exp2(zv) and u = 1 / (1 + t):
//   tanh z_v = 2 u - 1,   1 - tanh^2 z_v = 4 u (1 - u),
// so v = fma(u, c / 2, -c / 4) and s = fma(-u, u, u): 3 VALU + 2 transcendental instructions
// (v_exp_f32, v_rcp_f32) per value. t overflows to +inf for z_v < -44 (u = 0: tanh = -1,
// s = 0) and flushes to 0 for z_v > 44 (u = 1: tanh = 1, s = 0). Near tanh = +1, s carries the
// absolute rounding of u (about 6e-8), as 1 - a^2 does.
// The four values go in stages: the four exp2, then the four rcp, then the rest, with fences
// so the scheduler keeps the stages. Each value's chain is serial (exp2 -> add -> rcp -> fma),
// and left alone the compiler ran the chains one after another; a wave alone on its SIMD (the
// backward, the forward's last tiles) then waited out every transcendental's latency.
__device__ __forceinline__ void tanh_scaled4(const f4 zv, f4& v, f4& s) {
  f4 u;
#pragma unroll
  for (int r = 0; r < 4; ++r) u[r] = __builtin_amdgcn_exp2f(zv[r]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < 4; ++r) u[r] = __builtin_amdgcn_rcpf(u[r] + 1.0f);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    v[r] = __builtin_fmaf(u[r], 0.5f * kC, -0.25f * kC);
    s[r] = __builtin_fmaf(-u[r], u[r], u[r]);
  }
}

// tanh_jet of four values (component vectors z[c][r] of one accumulator row block), the tanh
// four at a time (tanh_scaled4): out[c][r] is the scaled output jet.
__device__ __forceinline__ void tanh_jet4(const f4 (&z)[4], f4 (&out)[4]) {
  f4 v, sl;
  tanh_scaled4(z[0], v, sl);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float q = __builtin_fmaf(z[1][r], z[1][r], z[2][r] * z[2][r]);
    out[0][r] = v[r];
    out[1][r] = sl[r] * z[1][r];
    out[2][r] = sl[r] * z[2][r];
    out[3][r] = sl[r] * __builtin_fmaf(v[r], q, z[3][r]);
  }
}

// Adjoint of the tanh jet (tanh_jet4, per value) in the scaled variables (the adjoint of a
// scaled quantity is the unscaled adjoint divided by the scale). With v' = (c / 4) tanh z_v,
// s' = s / 4, z'_J = 2 z_J, q' = |z'_J|^2, P = z'_L + v' q' and kappa = -8 / c^2 (so
// d s' / d(c z_v) = kappa v' s'):
//   zbar_v' = s' [vbar' + kappa v' (Jbar' . z'_J) + Lbar' (kappa v' P + s' q')]
//   zbar_Jd' = s' (Jbar_d' + 2 Lbar' v' z'_Jd)
//   zbar_L' = s' Lbar'
// the unscaled formulas with every quantity replaced by its scaled form (the factors cancel).
// This is the reference's tanh_backward (/root/reference/csrc/fused_backward.cu:29-33, 75-89)
// rewritten for the scaled jet. The adjoint (vbar', J0bar', J1bar', Lbar') is replaced in
// place. Evaluated as
//   zbar_L' = s' Lbar',   zbar_v' = s' [vbar' + kappa v' (Jbar' . z'_J + Lbar' P) + zbar_L' q'],
//   zbar_Jd' = s' Jbar_d' + 2 zbar_L' v' z'_Jd
// (17 instructions per value).
__device__ __forceinline__ void tanh_jet_adjoint_vs(float v, float s, float zj0, float zj1,
                                                    float zl, float& bv, float& bj0, float& bj1,
                                                    float& bl) {
  const float q = __builtin_fmaf(zj0, zj0, zj1 * zj1);
  const float dot = __builtin_fmaf(bj0, zj0, bj1 * zj1);
  const float p = __builtin_fmaf(v, q, zl);
  const float kv = kKappa * v;
  const float bls = bl * s;
  const float t = __builtin_fmaf(kv, __builtin_fmaf(bl, p, dot), bv);
  const float nv = s * __builtin_fmaf(bls, q, t);
  const float m2 = 2.0f * (bls * v);
  bj0 = __builtin_fmaf(m2, zj0, s * bj0);
  bj1 = __builtin_fmaf(m2, zj1, s * bj1);
  bv = nv;
  bl = bls;
}

// tanh_jet_adjoint_vs for layer 0, whose z_J are the W0 columns and z_L = 0: q = |z_J|^2 is
// the per-neuron constant staged in kSmallQ0 (the same fma), and p = v q.
__device__ __forceinline__ void tanh_jet_adjoint_layer0(float v, float s, float zj0, float zj1,
                                                        float q, float& bv, float& bj0,
                                                        float& bj1, float& bl) {
  const float dot = __builtin_fmaf(bj0, zj0, bj1 * zj1);
  const float p = v * q;
  const float kv = kKappa * v;
  const float bls = bl * s;
  const float t = __builtin_fmaf(kv, __builtin_fmaf(bl, p, dot), bv);
  const float nv = s * __builtin_fmaf(bls, q, t);
  const float m2 = 2.0f * (bls * v);
  bj0 = __builtin_fmaf(m2, zj0, s * bj0);
  bj1 = __builtin_fmaf(m2, zj1, s * bj1);
  bv = nv;
  bl = bls;
}

// An opaque copy of a value: the compiler cannot see that it equals the input, so it cannot
// hoist arithmetic on it (addresses, lane masks) out of the enclosing loop and keep the results
// live, where at full register use they would be spilled; and a loaded value passed through it
// is waited for there, not where the compiler would first use it.
template <typename T>
__device__ __forceinline__ T opaque(T x) {
  __asm__ volatile("" : "+v"(x));
  return x;
}

// Small-parameter staging shared by all kernels, in the scaled forms listed at kSmallCwx (the
// factors 2 and 4 are exact), split into its global loads (load_small) and its LDS writes
// (store_small), so that a kernel can issue these loads together with its other staging loads
// and wait for global memory once: written as one function, each group of loads waited for the
// previous group's LDS writes, and the forward's prologue made four round trips.
// Thread tid < 64 holds neuron tid's W0 row, b0 and w_out, thread tid < 192 one hidden bias,
// and every thread b_out (a uniform load).
struct SmallLoads {
  float wx, wy, b0, wo, bh, bout;
};

template <int kThreads>
__device__ __forceinline__ SmallLoads load_small(const float* __restrict__ params, int tid) {
  static_assert(kThreads >= 3 * kHidden, "one thread per hidden bias");
  SmallLoads s{0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (tid < kHidden) {
    s.wx = params[kInputs * tid];
    s.wy = params[kInputs * tid + 1];
    s.b0 = params[kLayer0Bias + tid];
    s.wo = params[kOutputBase + tid];
  }
  if (tid < 3 * kHidden) {
    s.bh = params[kHiddenBase + (tid >> 6) * kHiddenStride + kHidden * kHidden + (tid & 63)];
  }
  s.bout = params[kOutputBase + kHidden];
  return s;
}

// Called after the caller's other staging loads are issued. The values are waited for here: the
// opaque copies keep the compiler from moving the scaling up into load_small's branches, where
// it would wait for the loads at once.
__device__ __forceinline__ void store_small(float* s_small, int tid, SmallLoads s) {
  s.wx = opaque(s.wx);
  s.wy = opaque(s.wy);
  s.b0 = opaque(s.b0);
  s.wo = opaque(s.wo);
  s.bh = opaque(s.bh);
  s.bout = opaque(s.bout);
  if (tid < kHidden) {
    s_small[kSmallCwx + tid] = kC * s.wx;
    s_small[kSmallCwy + tid] = kC * s.wy;
    s_small[kSmallCb0 + tid] = kC * s.b0;
    s_small[kSmallWx + tid] = 2.0f * s.wx;
    s_small[kSmallWy + tid] = 2.0f * s.wy;
    s_small[kSmallQ0 + tid] = 4.0f * __builtin_fmaf(s.wx, s.wx, s.wy * s.wy);
    s_small[kSmallWoutV + tid] = 4.0f * (s.wo * (1.0f / kC));
    s_small[kSmallWoutL + tid] = 4.0f * (s.wo * (1.0f / kLambda));
  }
  if (tid < 3 * kHidden) s_small[kSmallBh + tid] = kC * s.bh;
  if (tid == 0) s_small[kSmallBout] = s.bout;
}

// Hidden-weight staging: every thread issues all of its global loads before its first LDS
// write (16-byte loads when the parameter buffer is 16-byte aligned, 4-byte loads otherwise),
// then scatters the values with put(layer, o, i, value) for W_layer[o][i].
template <int kThreads, typename Put>
__device__ __forceinline__ void stage_hidden(const float* __restrict__ params, int tid, Put put) {
  constexpr int kQuads = 3 * kHidden * kHidden / 4;
  constexpr int kPerThread = (kQuads + kThreads - 1) / kThreads;
  if ((reinterpret_cast<uintptr_t>(params) & 15) == 0) {
    f4 v[kPerThread];
#pragma unroll
    for (int n = 0; n < kPerThread; ++n) {
      const int q = tid + n * kThreads;
      if (q < kQuads) {
        const int layer = q >> 10, o = (q >> 4) & 63, i = (q & 15) << 2;
        v[n] = *reinterpret_cast<const f4*>(params + kHiddenBase + layer * kHiddenStride +
                                            (o << 6) + i);
      }
    }
#pragma unroll
    for (int n = 0; n < kPerThread; ++n) {
      const int q = tid + n * kThreads;
      if (q < kQuads) {
        const int layer = q >> 10, o = (q >> 4) & 63, i = (q & 15) << 2;
#pragma unroll
        for (int e = 0; e < 4; ++e) put(layer, o, i + e, v[n][e]);
      }
    }
  } else {
    for (int k = tid; k < 4 * kQuads; k += kThreads) {
      const int layer = k >> 12, o = (k >> 6) & 63, i = k & 63;
      put(layer, o, i, params[kHiddenBase + layer * kHiddenStride + (o << 6) + i]);
    }
  }
}

// Copy the packed parameters into LDS for the backward: the three hidden W, as 4 W (the scaled
// jet's weights), into pitch-68 planes, the small blocks in the scaled forms listed at
// kSmallCwx.
template <int kThreads>
__device__ __forceinline__ void stage_parameters(const float* __restrict__ params, float* s_w,
                                                 float* s_small, int tid) {
  const SmallLoads small = load_small<kThreads>(params, tid);
  stage_hidden<kThreads>(params, tid, [&](int layer, int o, int i, float value) {
    s_w[layer * kPlane + kWRow * o + i] = 4.0f * value;
  });
  store_small(s_small, tid, small);
}

// Forward-only LDS layout of the hidden weights, in MFMA operand order: for hidden layer l,
// k-step (ob, j) and lane (m, g), the 16 bytes at f4 index (16 l + 4 ob + j) * 64 + lane hold
// 4 W[16 mb + m][16 ob + 4 g + j] for mb = 0..3 (the scaled jet's weights). One ds_read_b128
// per k-step feeds the 4 MFMAs of that step; the 64 lanes read 1 KB contiguously (no bank
// conflicts) and every k-step offset is an instruction immediate.
constexpr int kOperandLayerF4 = 16 * kWave;  // f4 entries per layer (16 KB)

// Staging: work item (l, ob, lane) loads the 4 x 4 block of W_l with rows m, 16 + m, 32 + m,
// 48 + m and columns 16 ob + 4 g .. + 3 (four 16-byte global loads) and stores its 4 columns as
// the 4 k-steps (ob, j) of that lane: 16-byte LDS writes, each wave's 64 of them to 1 KB
// contiguous, so conflict-free. 768 work items: one per thread of a 12-wave workgroup, two for
// some threads of an 8-wave one; a thread issues the loads of all its items before its first
// LDS write.
template <int kThreads>
__device__ __forceinline__ void stage_operand_weights(const float* __restrict__ params, float* s_wa,
                                                      int tid) {
  constexpr int kItems = 3 * 4 * kWave;  // (layer, ob, lane)
  constexpr int kPerThread = (kItems + kThreads - 1) / kThreads;
  const bool aligned = (reinterpret_cast<uintptr_t>(params) & 15) == 0;
  f4* wa = reinterpret_cast<f4*>(s_wa);
  f4 rows[kPerThread][4];
#pragma unroll
  for (int n = 0; n < kPerThread; ++n) {
    const int item = tid + n * kThreads;
    if (item < kItems) {
      const int lane = item & (kWave - 1), ob = (item >> 6) & 3, layer = item >> 8;
      const float* block = params + kHiddenBase + layer * kHiddenStride + (lane & 15) * kHidden +
                           16 * ob + 4 * (lane >> 4);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const float* p = block + 16 * kHidden * mb;
        rows[n][mb] = aligned ? *reinterpret_cast<const f4*>(p) : f4{p[0], p[1], p[2], p[3]};
      }
    }
  }
#pragma unroll
  for (int n = 0; n < kPerThread; ++n) {
    const int item = tid + n * kThreads;
    if (item < kItems) {
      const int lane = item & (kWave - 1), ob = (item >> 6) & 3, layer = item >> 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        wa[(16 * layer + 4 * ob + j) * kWave + lane] =
            4.0f * f4{rows[n][0][j], rows[n][1][j], rows[n][2][j], rows[n][3][j]};
      }
    }
  }
}

// Layer-0 data of the 4 neurons o = 16 mb + 4 g + r (r = 0..3) held by this lane.
struct Layer0Weights {
  f4 cwx, cwy, cb;  // scaled, for the pre-activation c z_v = c (W0 x + b0)
  f4 wx, wy, q;     // z'_J0, z'_J1 of layer 0 (2 x the W0 columns) and their squared norm
};

__device__ __forceinline__ Layer0Weights layer0_weights(const float* s_small, int mb, int g) {
  const int o = 16 * mb + 4 * g;
  Layer0Weights w;
  w.cwx = lds4(s_small + kSmallCwx + o);
  w.cwy = lds4(s_small + kSmallCwy + o);
  w.cb = lds4(s_small + kSmallCb0 + o);
  w.wx = lds4(s_small + kSmallWx + o);
  w.wy = lds4(s_small + kSmallWy + o);
  w.q = lds4(s_small + kSmallQ0 + o);
  return w;
}

__device__ __forceinline__ float layer0_zv(const Layer0Weights& w, int r, float x0, float x1) {
  return __builtin_fmaf(w.cwx[r], x0, __builtin_fmaf(w.cwy[r], x1, w.cb[r]));
}

// Forward hidden product with the operand-native weight layout: wa points at this lane's f4
// in the layer's block; k-step (ob, j) reads wa[(4 ob + j) * 64]. Each k-step's operand is
// read one k-step ahead, with a fence on both sides of the step's 16 MFMAs so the read stays
// there: a wave that runs alone on its SIMD (the last tiles of a launch) then waits for no LDS
// read; left alone, the compiler issued each read right before its MFMAs. `first` = wa[0],
// read by the caller before the previous layer's tanh jet.
__device__ __forceinline__ void hidden_product_native(const f4* wa, const f4 (&h)[4][4],
                                                      const f4 (&bias)[4], f4 (&acc)[4][4],
                                                      f4 first) {
  f4 next = first;
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int step = 4 * ob + j;
      const f4 a = next;
      if (step < 15) next = wa[(step + 1) * kWave];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f4 cin = (ob | j) ? acc[mb][c] : (c == 0 ? bias[mb] : f4{0.f, 0.f, 0.f, 0.f});
          acc[mb][c] = mfma(a[mb], h[ob][c][j], cin);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Scaled value biases c b of the 4 x 4 neurons 16 mb + 4 g + r held by this lane.
__device__ __forceinline__ void load_bias(const float* s_small, int layer, int g, f4 (&bias)[4]) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) bias[mb] = lds4(s_small + kSmallBh + layer * kHidden + 16 * mb + 4 * g);
}

// tanh_jet over a layer's 16 values per lane, the tanh four at a time (tanh_scaled4).
__device__ __forceinline__ void apply_tanh_jet(const f4 (&z)[4][4], f4 (&h)[4][4]) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    f4 v, sl;
    tanh_scaled4(z[mb][0], v, sl);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float zj0 = z[mb][1][r], zj1 = z[mb][2][r];
      const float q = __builtin_fmaf(zj0, zj0, zj1 * zj1);
      h[mb][0][r] = v[r];
      h[mb][1][r] = sl[r] * zj0;
      h[mb][2][r] = sl[r] * zj1;
      h[mb][3][r] = sl[r] * __builtin_fmaf(v[r], q, z[mb][3][r]);
    }
  }
}

// Layer 0 in closed form: the input jet is (x, I, 0), so z_J = W0 columns and z_L = 0, and
// the tanh jet's q = |z_J|^2 is a per-neuron constant.
// One block: the jet of neurons 16 mb + 4 g + r, r = 0..3, in h[c][r].
__device__ __forceinline__ void layer0_block(const float* s_small, int mb, int g, float x0,
                                             float x1, f4 (&h)[4]) {
  const Layer0Weights w = layer0_weights(s_small, mb, g);
  f4 zv, v, s;
#pragma unroll
  for (int r = 0; r < 4; ++r) zv[r] = layer0_zv(w, r, x0, x1);
  tanh_scaled4(zv, v, s);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    h[0][r] = v[r];
    h[1][r] = s[r] * w.wx[r];
    h[2][r] = s[r] * w.wy[r];
    h[3][r] = s[r] * (v[r] * w.q[r]);
  }
}

__device__ __forceinline__ void layer0_forward(const float* s_small, int g, float x0, float x1,
                                               f4 (&h)[4][4]) {
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) layer0_block(s_small, mb, g, x0, x1, h[mb]);
}

// The small LDS parameters read per tile have loop-invariant addresses; left alone, the
// compiler hoists those reads out of the tile loop and keeps ~100 values live in registers for
// the whole kernel. An empty asm statement with a memory clobber at the top of each tile keeps
// them as per-tile LDS reads.
__device__ __forceinline__ void keep_lds_reads_in_loop() { __asm__ volatile("" ::: "memory"); }

// A scheduling fence that only SALU instructions cross. Placed between the LDS reads for the
// next step and the MFMAs of the current one, it keeps the reads issued a step ahead (at full
// register use the scheduler otherwise sinks each read to just before its first use, and the
// MFMA then waits out the LDS latency). It also keeps VALU work out of the MFMA runs: FP32
// MFMA and VALU never execute together on gfx950, and a VALU instruction issued right after an
// MFMA costs about 8 cycles more than one issued after another VALU instruction (measured with
// a one-wave probe: 1 MFMA + k independent FMAs take 32.5 + 8 + 4.7 k cycles, 4 MFMAs + 16
// FMAs no more than their separate times). Letting VALU cross, the scheduler had spread single
// instructions between MFMAs, about 250 such switches per backward tile; with this fence 57.
__device__ __forceinline__ void lds_mfma_fence() { __builtin_amdgcn_sched_barrier(0x0004); }

// Value of lane l ^ 32 (permlane32) or l ^ 16 (permlane16) in every lane, with gfx950's
// v_permlane32_swap / v_permlane16_swap (VALU, no LDS round trip). swap(u, 0) leaves the
// partner in .second of the low half, swap(0, u) in .first of the high half, and the other
// halves are zero. (Swapping a register with a copy of itself would need one swap, but the
// compiler folds that form to the wrong result.)
__device__ __forceinline__ float partner32(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto a = __builtin_amdgcn_permlane32_swap(u, 0u, false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(0u, u, false, false);
  return __builtin_bit_cast(float, a[1] | b[0]);
}

__device__ __forceinline__ float partner16(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, 0u, false, false);
  const auto b = __builtin_amdgcn_permlane16_swap(0u, u, false, false);
  return __builtin_bit_cast(float, a[1] | b[0]);
}

// x[l] + x[l ^ 32] + x[l ^ 16] + x[l ^ 48] in every lane, bitwise identical across the four
// lanes (each pairwise sum adds the same two operands).
__device__ __forceinline__ float sum_lane_groups(float x) {
  const float y = x + partner32(x);
  return y + partner16(y);
}

// Sum over the 16 lanes of a row (lanes 16 g .. 16 g + 15), identical in all 16 lanes: DPP
// butterflies xor 1 and xor 2 (quad_perm), then the 8- and 16-lane mirrors.
__device__ __forceinline__ float sum_row16(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x140, 0xF, 0xF, true));
  return x;
}

template <int kCtrl>
__device__ __forceinline__ float dpp_read(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, true));
}

// Reduce-scatter over the 16 lanes of a row: lane m of the row (m = lane % 16) returns the sum
// of v[m] over the row's lanes. Four butterfly stages, with partners given by DPP: the row
// mirror (lane 15 - m), the half-row mirror (7 - m within each 8), then quad xor 2 and xor 1.
// At each stage a lane keeps the half of its partial sums whose indices it or its remaining
// partners will own and adds the partner's copy of that half, so the work halves per stage:
// 45 VALU instructions, against 80 for 16 full row sums and picks.
__device__ __forceinline__ float row_reduce_scatter16(const float (&v)[16], int m) {
  const bool b3 = (m & 8) != 0, b2 = (m & 4) != 0, b1 = (m & 2) != 0, b0 = (m & 1) != 0;
  float s8[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float keep = b3 ? v[j + 8] : v[j];
    const float send = b3 ? v[j] : v[j + 8];
    s8[j] = keep + dpp_read<0x140>(send);
  }
  float s4[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float keep = b2 ? s8[k + 4] : s8[k];
    const float send = b2 ? s8[k] : s8[k + 4];
    s4[k] = keep + dpp_read<0x141>(send);
  }
  float s2[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const float keep = b1 ? s4[k + 2] : s4[k];
    const float send = b1 ? s4[k] : s4[k + 2];
    s2[k] = keep + dpp_read<0x4E>(send);
  }
  const float keep = b0 ? s2[1] : s2[0];
  const float send = b0 ? s2[0] : s2[1];
  return keep + dpp_read<0xB1>(send);
}

// ---------------------------------------------------------------------------------------------
// Layer outputs saved by the forward for a backward that reads them instead of re-running the
// forward (fhoad_forward_laplacian_saving, fhoad_forward_laplacian_backward_saved): per
// 16-point tile t, hidden layer l (0..2 for layers 1..3), row block mb and jet component c, the
// 64 lanes' f4 in lane order. Lane (m, g)'s f4 holds rows 16 mb + 4 g + r (r = 0..3) at point
// 16 t + m, the MFMA accumulator layout every kernel here keeps a layer's output in, so each
// store and load moves 1 KB per wave contiguously. 3,072 f4 (49,152 bytes) per tile.
constexpr int64_t kSavedF4PerTile = 3 * 16 * kWave;
__device__ __forceinline__ int64_t saved_index(int64_t tile, int layer, int mb, int c, int lane) {
  return ((tile * 3 + layer) * 16 + 4 * mb + c) * kWave + lane;
}

// The forward writes the saved layers as non-temporal stores (about 2 us less per 64K call than
// plain stores, measured); the backward reads them with plain loads (non-temporal loads
// measured about 7 us slower per 64K call).
__device__ __forceinline__ void store_saved(f4* __restrict__ saved, int64_t index, f4 value) {
  __builtin_nontemporal_store(value, &saved[index]);
}

// One hidden layer's saved output of a 16-point tile into the accumulator layout (zeros for a
// tile past the saved ones).
__device__ __forceinline__ void load_saved_layer(const f4* __restrict__ saved, int64_t tile,
                                                 int64_t saved_tiles, int layer, int lane,
                                                 f4 (&h)[4][4]) {
  if (tile < saved_tiles) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int c = 0; c < 4; ++c) h[mb][c] = saved[saved_index(tile, layer, mb, c, lane)];
    }
  } else {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
      for (int c = 0; c < 4; ++c) h[mb][c] = f4{0.f, 0.f, 0.f, 0.f};
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Forward kernel (replaces fused_forward_laplacian_tiled_kernel<2>,
// /root/reference/csrc/fused_residual.cu:157-295). A grid of at most one workgroup per CU
// stages the weights once, then every wave walks 16-point tiles: tile t < whole goes to
// workgroup t % grid, wave (t / grid) % kWaves, so small batches still spread over all CUs.
//
// `whole` is a multiple of 4 x grid (one tile per SIMD per round), so every SIMD runs the same
// number of whole tiles. The tiles past the last whole round (`split` tiles, fewer than one per
// SIMD) would each add a whole tile's time to the SIMD that got it; instead, the last four
// waves of each workgroup (one per SIMD, the ones with the fewest whole tiles) run them with a
// 16-point tile's rows split between them, forward_split_kernel's decomposition: wave q
// computes rows 16 q .. 16 q + 15 of every layer (64 MFMAs per layer instead of 256) and the
// layer outputs go to the other three through LDS. The four meet at an LDS counter
// (quad_sync), not at s_barrier, which would wait for the workgroup's waves still on whole
// tiles. A split tile's chains are a whole tile's accumulators (mb = q, c) with the same
// operands in the same order, so both paths give bitwise the same results.
constexpr int kQuadSpinLimit = 1 << 24;  // about 0.5 s of s_sleep(1); never reached by a whole quad

// Device status word, one per GPU: bit kStatusQuadTimeout is set when a quad meeting gave up
// (quad_sync below). fhoad_check_device reads and clears it.
constexpr unsigned kStatusQuadTimeout = 1u;
__device__ unsigned g_device_status = 0;

// The four waves of a quad each add 1 to `flag` per meeting and wait until it reaches `target`
// (4 x the meetings so far), polling at most `spin_limit` times. The release fence completes the
// wave's LDS writes before its arrival; the acquire fence orders its later reads after the
// others' arrivals. Every quad wave takes the same split tiles and meetings, so the wait ends;
// the limit only bounds it. Returns false when the wave gave up: it then sets
// kStatusQuadTimeout in the device status word (a global atomic OR) and goes on, and the caller
// writes NaN for that tile's u and Laplacian.
__device__ __forceinline__ bool quad_sync(unsigned* flag, unsigned target, int spin_limit) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  if ((threadIdx.x & (kWave - 1)) == 0) {
    __hip_atomic_fetch_add(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  bool met = false;
  for (int spin = 0; spin < spin_limit; ++spin) {
    if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) {
      met = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (!met && (threadIdx.x & (kWave - 1)) == 0) {
    __hip_atomic_fetch_or(&g_device_status, kStatusQuadTimeout, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT);
  }
  return met;
}

// kSave: also write each tile's hidden-layer outputs to `saved` (saved_index).
template <int kWaves, bool kSave>
__global__ void __launch_bounds__(kWaves * kWave)
forward_kernel(const float* __restrict__ coordinates, const float* __restrict__ params,
               float* __restrict__ output, float* __restrict__ laplacian, int64_t batch,
               int64_t whole, int64_t tiles, f4* __restrict__ saved, int spin_limit) {
  __shared__ __attribute__((aligned(16))) float s_wa[3 * kOperandLayerF4 * 4];
  __shared__ __attribute__((aligned(16))) float s_small[kSmallFloats];
  __shared__ f4 s_x[2][4][4][kWave];  // split tiles: [buffer][wave q][component][lane], 32 KB
  __shared__ unsigned s_quad;         // split tiles: quad_sync counter
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int g = lane >> 4;
  const int m = lane & 15;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kWaves;
  // Coordinates are read one tile ahead (the first tile's during the staging), so no tile
  // waits for global memory; a wave that runs alone on its SIMD would expose that latency.
  int64_t tile = blockIdx.x + static_cast<int64_t>(wave) * gridDim.x;
  float next_x0 = 0.0f, next_x1 = 0.0f;
  if (tile < whole && tile * kTile + m < batch) {
    next_x0 = coordinates[2 * (tile * kTile + m)];
    next_x1 = coordinates[2 * (tile * kTile + m) + 1];
  }
  if (threadIdx.x == 0) s_quad = 0;
  const SmallLoads small = load_small<kWaves * kWave>(params, threadIdx.x);
  stage_operand_weights<kWaves * kWave>(params, s_wa, threadIdx.x);
  store_small(s_small, threadIdx.x, small);
  __syncthreads();
  next_x0 = opaque(next_x0);  // delivered before the loop, for the same reason as below
  next_x1 = opaque(next_x1);

  // ---- split tiles first: the last four waves, one 16-point tile at a time, rows split ----
  // (first, so their quarter tiles interleave with the other waves' whole tiles on each SIMD)
  const int q = wave - (kWaves - 4);
  if (q >= 0 && whole < tiles) {
    // Raised wave priority while on split tiles: the four waves of a quad meet three times a
    // tile, each meeting waits for the slowest of them, and each shares its SIMD with two waves
    // on whole tiles. (65,537 points: 54.9 -> 53.5 us per call, 70,000: 60.6 -> 57.7 us,
    // 100,000: 79.8 -> 78.5 us; levels 1 to 3 measured the same.)
    __builtin_amdgcn_s_setprio(2);
    const float* wa_q = s_wa + 4 * lane + q;  // component q of this lane's operand f4s
    unsigned meetings = 0;
    int phase = 0;  // alternates the exchange buffers across layers and tiles
    for (int64_t t = whole + blockIdx.x; t < tiles; t += gridDim.x) {
      keep_lds_reads_in_loop();
      const int64_t point = t * kTile + m;
      const bool active = point < batch;
      float x0 = 0.0f, x1 = 0.0f;
      if (active) {
        x0 = coordinates[2 * point];
        x1 = coordinates[2 * point + 1];
      }
      f4 h[4][4];
      layer0_forward(s_small, g, x0, x1, h);
      bool met = true;  // every quad meeting of this tile completed
#pragma unroll
      for (int layer = 0; layer < 3; ++layer) {
        const f4 bias = lds4(s_small + kSmallBh + layer * kHidden + 16 * q + 4 * g);
        f4 acc[4];
#pragma unroll
        for (int ob = 0; ob < 4; ++ob) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            // 4 W[16 q + m][16 ob + 4 g + j]: component q of k-step (ob, j)'s operand f4
            const float a = wa_q[4 * ((16 * layer + 4 * ob + j) * kWave)];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              const f4 cin = (ob | j) ? acc[c] : (c == 0 ? bias : f4{0.f, 0.f, 0.f, 0.f});
              acc[c] = mfma(a, h[ob][c][j], cin);
            }
          }
        }
        f4 mine[4];
        tanh_jet4(acc, mine);
        if (kSave) {
#pragma unroll
          for (int c = 0; c < 4; ++c) store_saved(saved, saved_index(t, layer, q, c, lane), mine[c]);
        }
        f4 (*buf)[4][kWave] = s_x[phase];
        phase ^= 1;
#pragma unroll
        for (int c = 0; c < 4; ++c) buf[q][c][lane] = mine[c];
        meetings += 4;
        met = quad_sync(&s_quad, meetings, spin_limit) && met;
        if (layer < 2 || q == 0) {  // after the last layer only wave q = 0 (the output) reads
#pragma unroll
          for (int ob = 0; ob < 4; ++ob) {
#pragma unroll
            for (int c = 0; c < 4; ++c) h[ob][c] = buf[ob][c][lane];
          }
        }
      }
      if (q == 0) {
        float u = 0.0f, lap = 0.0f;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          const f4 wv = lds4(s_small + kSmallWoutV + 16 * mb + 4 * g);
          const f4 wl = lds4(s_small + kSmallWoutL + 16 * mb + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            u = __builtin_fmaf(wv[r], h[mb][0][r], u);
            lap = __builtin_fmaf(wl[r], h[mb][3][r], lap);
          }
        }
        u = sum_lane_groups(u);
        lap = sum_lane_groups(lap);
        if (g == 0 && active) {
          // A tile whose meetings gave up read stale rows: its outputs are NaN (and the device
          // status word says why).
          output[point] = met ? u + s_small[kSmallBout] : __builtin_nanf("");
          laplacian[point] = met ? lap : __builtin_nanf("");
        }
      }
    }
  }

  __builtin_amdgcn_s_setprio(0);
  const f4* wa_lane = reinterpret_cast<const f4*>(s_wa) + lane;
  for (; tile < whole; tile += step) {
    keep_lds_reads_in_loop();
    const int64_t point = tile * kTile + m;
    const bool active = point < batch;
    const float x0 = next_x0, x1 = next_x1;
    const int64_t next_point = (tile + step) * kTile + m;
    if (tile + step < whole && next_point < batch) {
      next_x0 = coordinates[2 * next_point];
      next_x1 = coordinates[2 * next_point + 1];
    }
    f4 first = wa_lane[0];
    f4 h[4][4];
    layer0_forward(s_small, g, x0, x1, h);
    for (int layer = 0; layer < 3; ++layer) {
      f4 bias[4];
      load_bias(s_small, layer, g, bias);
      f4 acc[4][4];
      hidden_product_native(wa_lane + layer * kOperandLayerF4, h, bias, acc, first);
      if (layer < 2) first = wa_lane[(layer + 1) * kOperandLayerF4];
      apply_tanh_jet(acc, h);
      if (kSave) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
          for (int c = 0; c < 4; ++c) store_saved(saved, saved_index(tile, layer, mb, c, lane), h[mb][c]);
        }
      }
    }
    // Take delivery of the next coordinates here, before this tile's stores: a wait at the
    // top of the next tile would also wait for those stores (they sit behind a branch, so the
    // compiler cannot count them), and a store takes far longer than a tile's head.
    next_x0 = opaque(next_x0);
    next_x1 = opaque(next_x1);
    // u = w_out . v + b_out and lap = w_out . L, from the scaled jet.
    float u = 0.0f, lap = 0.0f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const f4 wv = lds4(s_small + kSmallWoutV + 16 * mb + 4 * g);
      const f4 wl = lds4(s_small + kSmallWoutL + 16 * mb + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        u = __builtin_fmaf(wv[r], h[mb][0][r], u);
        lap = __builtin_fmaf(wl[r], h[mb][3][r], lap);
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
// Small-batch forward. With fewer tiles than SIMDs, forward_kernel's call time is one tile's
// latency: 768 dependent MFMAs on one wave. Here a workgroup of 4 waves (one per SIMD) runs one
// 16-point tile at a time, and wave w computes output rows 16 w .. 16 w + 15 of every layer
// (64 MFMAs per layer instead of 256). The tanh-jet outputs go through LDS to the other waves,
// which need all 64 rows as the next layer's B operand. In forward_kernel's register layout the
// B operand of k-step (ob, j) is register j of accumulator (ob, c) of the same lane, so the
// exchange is lane to lane: each wave stores its 4 f4 per lane and reads the other waves' f4
// at the same lane index (1 KB contiguous per wave access, no bank conflicts). Two LDS buffers
// alternate, so one barrier per layer suffices.
//
// Wave w's chains are forward_kernel's accumulators (mb = w, c) with the same operands in the
// same order, layer 0 is the same closed form, and wave 0 forms u and lap in forward_kernel's
// order, so both kernels give bitwise the same results.
constexpr int kSplitWaves = 4;

template <bool kSave>
__global__ void __launch_bounds__(kSplitWaves * kWave)
forward_split_kernel(const float* __restrict__ coordinates, const float* __restrict__ params,
                     float* __restrict__ output, float* __restrict__ laplacian, int64_t batch,
                     int64_t tiles, f4* __restrict__ saved) {
  __shared__ f4 s_h[2][kSplitWaves][4][kWave];  // [buffer][wave][component][lane], 32 KB
  __shared__ __attribute__((aligned(16))) float s_small[kSmallFloats];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int m = lane & 15;
  const int g = lane >> 4;
  // The small parameters are staged first and this wave's operands loaded after (they are needed
  // only after the barrier and the first tile's coordinates): issued together, the operand loads
  // were waited for before the barrier and a 1K-point call took 0.4 us longer.
  store_small(s_small, threadIdx.x, load_small<kSplitWaves * kWave>(params, threadIdx.x));
  // A operands of this wave's rows: wa[l][ob][j] = 4 W_l[16 w + m][16 ob + 4 g + j] (the
  // scaled jet's weights), loaded once (global memory, L2-resident) instead of staging
  // the whole matrix in LDS.
  f4 wa[3][4];
  {
    const float* row = params + kHiddenBase + (16 * w + m) * kHidden + 4 * g;
    const bool aligned = (reinterpret_cast<uintptr_t>(params) & 15) == 0;
#pragma unroll
    for (int l = 0; l < 3; ++l) {
#pragma unroll
      for (int ob = 0; ob < 4; ++ob) {
        const float* p = row + l * kHiddenStride + 16 * ob;
        wa[l][ob] = 4.0f * (aligned ? *reinterpret_cast<const f4*>(p) : f4{p[0], p[1], p[2], p[3]});
      }
    }
  }
  __syncthreads();  // s_small

  int phase = 0;  // alternates the exchange buffers across layers and tiles
  for (int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    keep_lds_reads_in_loop();
    const int64_t point = tile * kTile + m;
    const bool active = point < batch;
    float x0 = 0.0f, x1 = 0.0f;
    if (active) {
      x0 = coordinates[2 * point];
      x1 = coordinates[2 * point + 1];
    }
    f4 h[4][4];
    layer0_forward(s_small, g, x0, x1, h);
#pragma unroll
    for (int layer = 0; layer < 3; ++layer) {
      const f4 bias = lds4(s_small + kSmallBh + layer * kHidden + 16 * w + 4 * g);
      f4 acc[4];
#pragma unroll
      for (int ob = 0; ob < 4; ++ob) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const f4 cin = (ob | j) ? acc[c] : (c == 0 ? bias : f4{0.f, 0.f, 0.f, 0.f});
            acc[c] = mfma(wa[layer][ob][j], h[ob][c][j], cin);
          }
        }
      }
      f4 mine[4];
      {
        f4 v, sl;
        tanh_scaled4(acc[0], v, sl);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float q = __builtin_fmaf(acc[1][r], acc[1][r], acc[2][r] * acc[2][r]);
          mine[0][r] = v[r];
          mine[1][r] = sl[r] * acc[1][r];
          mine[2][r] = sl[r] * acc[2][r];
          mine[3][r] = sl[r] * __builtin_fmaf(v[r], q, acc[3][r]);
        }
      }
      if (kSave) {
#pragma unroll
        for (int c = 0; c < 4; ++c) store_saved(saved, saved_index(tile, layer, w, c, lane), mine[c]);
      }
      f4 (*buf)[4][kWave] = s_h[phase];
      phase ^= 1;
#pragma unroll
      for (int c = 0; c < 4; ++c) buf[w][c][lane] = mine[c];
      __syncthreads();
      if (layer < 2 || w == 0) {  // after the last layer only wave 0 (the output) reads
#pragma unroll
        for (int ob = 0; ob < 4; ++ob) {
#pragma unroll
          for (int c = 0; c < 4; ++c) h[ob][c] = ob == w ? mine[c] : buf[ob][c][lane];
        }
      }
    }
    if (w == 0) {
      float u = 0.0f, lap = 0.0f;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const f4 wv = lds4(s_small + kSmallWoutV + 16 * mb + 4 * g);
        const f4 wl = lds4(s_small + kSmallWoutL + 16 * mb + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          u = __builtin_fmaf(wv[r], h[mb][0][r], u);
          lap = __builtin_fmaf(wl[r], h[mb][3][r], lap);
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
}

// ---------------------------------------------------------------------------------------------
// Backward (replaces fused_backward_occupancy_kernel<false,true,false,true> and the host-side
// partials.sum(0), /root/reference/csrc/fused_backward.cu:424-850, 859-934).
//
// One workgroup per CU, 4 waves (one per SIMD, up to 512 registers each), 64-point workgroup
// tiles (16 points per wave). Per tile:
//   1. every wave re-runs the forward for its 16 points, keeping each hidden layer's tanh-jet
//      output h in registers;
//   2. the adjoint is seeded from the linear output layer and walked back through layers 3..1:
//      tanh-jet adjoint from h in registers (tanh_jet_adjoint_h, no tanh re-evaluated),
//      dW += zbar h_prev^T, hbar = W^T zbar one input block at a time (registers), and
//      finally layer 0 in closed form;
//   3. dW contracts over the points of all 4 waves: zbar and h_prev are staged in LDS (three
//      jet components written behind the MFMAs of the phase before, the fourth behind the first
//      components' dW MFMAs; see staged_dw) and wave w owns output rows 16 w .. 16 w + 15 of
//      every dW; the hidden bias gradients fall out of the same LDS reads. W0, b0 and w_out gradients are
//      summed over each wave's points in registers (row_reduce_scatter16) and over the 4 waves once
//      per slot.
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

// Staging bases of one lane, formed where each phase starts (from opaque copies of the lane
// offsets, see backward_kernel): writes of zbar (planes 0..2) and h_prev (planes 3..5) at rows
// 4 g + r of a block and point 16 w + m; reads of the A operand (this wave's rows 16 w + m, zbar
// planes) and of the B operands (rows 16 n + m, h_prev planes) at points 4 g .. 4 g + 3 of a
// 16-point block. Every other offset is an instruction immediate (planes 0..2 from a base stay
// within a DS offset's 64 KB reach, hence the second base for planes 3..5).
struct StageBases {
  float* wz;
  float* wh;
  const float* ra;
  const float* rb;
};

// Staging write i (0..23) of block mb: the three early components of zbar (x, planes 0..2) and
// of h_prev (y, planes 3..5), alternating, for this lane's rows 16 mb + 4 g + r.
__device__ __forceinline__ void stage_early_write(const StageBases& sb, int mb, const f4 (&x)[4],
                                                  const f4 (&y)[4], int i) {
  const int e = i >> 3, r = (i >> 1) & 3;
  float* base = (i & 1) ? sb.wh : sb.wz;
  base[e * kPlane + kWRow * (16 * mb + r)] = (i & 1) ? y[early_component(e)][r] : x[early_component(e)][r];
}

// Staging write i (0..31) of the late component: zbar (xl[mb], plane 0) and h_prev (yl[mb],
// plane 3), alternating, rows 16 mb + 4 g + r.
__device__ __forceinline__ void stage_late_write(const StageBases& sb, const f4 (&xl)[4],
                                                 const f4 (&yl)[4], int i) {
  const int mb = i >> 3, r = (i >> 1) & 3;
  float* base = (i & 1) ? sb.wh : sb.wz;
  base[kWRow * (16 * mb + r)] = (i & 1) ? yl[mb][r] : xl[mb][r];
}

// The five 16-byte operands of one dW step: the A operand zbar[16 w + m][p] and the B operands
// h_prev[16 n + m][p], n = 0..3, for p = 16 s + 4 g + k, k = 0..3, of the component staged in
// plane pair (plane, 3 + plane).
struct DwOperands {
  f4 a, b[4];
};

__device__ __forceinline__ DwOperands dw_read(const StageBases& sb, int plane, int s) {
  DwOperands o;
  o.a = lds4(sb.ra + plane * kPlane + 16 * s);
#pragma unroll
  for (int n = 0; n < 4; ++n) o.b[n] = lds4(sb.rb + plane * kPlane + 16 * kWRow * n + 16 * s);
  return o;
}

// dW[16 w + ., 16 n + .] += sum over the 64 tile points of zbar_c h_prev_c^T for the components
// staged in plane pairs (kFirst + i, kFirst + 3 + i), i < kN: four steps (point blocks) per
// component, 16 MFMAs each contracting over the step's points; every lane supplies the same
// points at each step. `ops` holds the first step's operands on entry and each step reads the
// next step's; with kNext >= 0 the last step reads the first operands of plane pair kNext into
// `ops`. emit(step, k) issues staging writes after the MFMAs of point k: they follow the next
// step's reads, so waiting for those reads never waits for them, and they drain behind the
// MFMAs. With kBias, returns the sum of this lane's reads of the first component (the hidden bias
// gradient's partial for row 16 w + m when it is zbar_v).
template <int kFirst, int kN, bool kBias, int kNext, typename Emit>
__device__ __forceinline__ float dw_pass(const StageBases& sb, DwOperands& ops, f4 (&dw)[4],
                                         Emit emit) {
  float bias = 0.0f;
#pragma unroll
  for (int step = 0; step < 4 * kN; ++step) {
    const DwOperands cur = ops;
    if (kBias && step < 4) {
#pragma unroll
      for (int k = 0; k < 4; ++k) bias += cur.a[k];
    }
    if (step + 1 < 4 * kN) {
      ops = dw_read(sb, kFirst + ((step + 1) >> 2), (step + 1) & 3);
    } else if (kNext >= 0) {
      ops = dw_read(sb, kNext, 0);
    }
    lds_mfma_fence();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
      for (int n = 0; n < 4; ++n) dw[n] = mfma(cur.a[k], cur.b[n][k], dw[n]);
      if (emit(step, k)) __builtin_amdgcn_sched_barrier(0);
    }
    lds_mfma_fence();
  }
  return bias;
}

// emit() that issues nothing.
struct NoEmit {
  __device__ __forceinline__ bool operator()(int, int) const { return false; }
};

// after() that does nothing.
struct NoAfter {
  __device__ __forceinline__ void operator()(int) const {}
};

// Per-neuron sums over a wave's 16 points without LDS: lane (m, g) holds x for neuron
// 16 mb + 4 g + r at point m, so summing value k = 4 mb + r over the 16 lanes of row g gives
// that neuron's total; row_reduce_scatter16 leaves the total of k = m in lane m. Lane (m, g)
// thus keeps the total of neuron owned_neuron(m, g) = 16 (m >> 2) + 4 g + (m & 3): the 64 lanes
// own the 64 neurons once each.
__device__ __forceinline__ int owned_neuron(int m, int g) { return 16 * (m >> 2) + 4 * g + (m & 3); }

// dW += zbar h_prev^T over the workgroup tile from the staged planes, once the early components
// of zbar and h_prev are written (planes 0..2, 3..5) and the late ones are in registers (xl: zbar,
// yl: h_prev, per block):
//   barrier; component e = 0 (zbar_v: the bias sum); barrier (every wave is done with planes 0
//   and 3); components e = 1, 2, with the late component's writes into planes 0 and 3 between
//   their MFMAs; barrier; the late component.
// Adds sum_p zbar_v' of row 16 w + m (all lane groups) to g_bias. The products accumulate in the
// component order v, L, J0, J1 and point order of each, as two passes of (v, L), (J0, J1) did.
__device__ __forceinline__ void staged_dw(const StageBases& sb, const f4 (&xl)[4], const f4 (&yl)[4],
                                          f4 (&dw)[4], float& g_bias) {
  __syncthreads();  // the early components are written
  DwOperands ops = dw_read(sb, 0, 0);
  // The first pass's last step reads the second pass's first operands (planes 1 and 4 were
  // complete at the first barrier), so the second pass does not start by waiting for LDS.
  g_bias += sum_lane_groups(dw_pass<0, 1, true, 1>(sb, ops, dw, NoEmit{}));
  __syncthreads();  // every wave is done with planes 0 and 3
  dw_pass<1, 2, false, -1>(sb, ops, dw, [&](int step, int k) {
    stage_late_write(sb, xl, yl, 4 * step + k);
    return true;
  });
  __syncthreads();  // the late component is written
  ops = dw_read(sb, 0, 0);
  dw_pass<0, 1, false, -1>(sb, ops, dw, NoEmit{});
}

// ---- the interior tiles of backward_kernel: the walk back from each layer's tanh-jet output ----
//
// The adjoint of the tanh jet (tanh_jet_adjoint_vs) needs s', z'_J and P = z'_L + v' q' only
// in the products the jet's output already holds: h' = (v', s' z'_J0, s' z'_J1, s' P), so
// s' z'_J = h'_J, s' P = h'_L and s'^2 q' = |h'_J|^2. With s' from v' alone,
//   s' = 1/4 + (kappa / 2) v'^2      (v' = (c / 4) tanh z_v, kappa = -8 / c^2: (1 - tanh^2) / 4),
// the adjoint is
//   zbar_L' = s' Lbar',   zbar_Jd' = s' Jbar_d' + 2 Lbar' v' h'_Jd,
//   zbar_v' = s' vbar' + kappa v' (Jbar' . h'_J + Lbar' h'_L) + Lbar' |h'_J|^2
// (18 instructions per value). A tile therefore keeps each hidden layer's output h (which the
// forward re-run produces anyway, and which the weight gradient of the layer above needs) and
// evaluates no tanh in the walk back. Near |tanh| = 1, s' carries an absolute rounding of about
// 3e-8, as 1 - a^2 does in the reference (/root/reference/csrc/fused_backward.cu:65-89).
constexpr float kHalfKappa = 0.5f * kKappa;

__device__ __forceinline__ void tanh_jet_adjoint_h(float v, float hj0, float hj1, float hl,
                                                   float& bv, float& bj0, float& bj1, float& bl) {
  const float hk = kHalfKappa * v;
  const float s = __builtin_fmaf(hk, v, 0.25f);
  const float kv = hk + hk;
  const float lv2 = bl * (v + v);
  const float dot = __builtin_fmaf(bj0, hj0, bj1 * hj1);
  const float q = __builtin_fmaf(hj0, hj0, hj1 * hj1);
  const float t = __builtin_fmaf(bl, hl, dot);
  const float nv = __builtin_fmaf(bl, q, __builtin_fmaf(kv, t, s * bv));
  bj0 = __builtin_fmaf(lv2, hj0, s * bj0);
  bj1 = __builtin_fmaf(lv2, hj1, s * bj1);
  bv = nv;
  bl = s * bl;
}

// tanh_jet_adjoint_h for the output layer's seed: Jbar' = 0 and, with kZeroV (interior points
// of the fused step), vbar' = 0; only operations on those zeros are dropped.
template <bool kZeroV>
__device__ __forceinline__ void tanh_jet_adjoint_h_seed(float v, float hj0, float hj1, float hl,
                                                        float& bv, float& bj0, float& bj1,
                                                        float& bl) {
  const float hk = kHalfKappa * v;
  const float s = __builtin_fmaf(hk, v, 0.25f);
  const float kv = hk + hk;
  const float lv2 = bl * (v + v);
  const float q = __builtin_fmaf(hj0, hj0, hj1 * hj1);
  const float t = bl * hl;
  const float w = kZeroV ? kv * t : __builtin_fmaf(kv, t, s * bv);
  bv = __builtin_fmaf(bl, q, w);
  bj0 = lv2 * hj0;
  bj1 = lv2 * hj1;
  bl = s * bl;
}

// One hidden layer of the forward re-run, one output block at a time: z = W[16 mb + ., :] h_in
// + b (the first k-step takes the bias as its C operand), then the block's tanh jet into
// h_out[mb]. Each accumulator takes its k-steps (ob, j) in order (as in forward_kernel's
// hidden_product_native); a block's tanh jet (VALU) and the next block's 64 MFMAs are independent,
// so either can fill the other's latencies. The next block's four A operands (16-byte LDS
// reads) are issued before this block's MFMAs, so no block waits for LDS. w_rows is this
// lane's row base (68 m + 4 g). emit(mb, k) may issue LDS writes after k-step k (0..15) of
// block mb's MFMAs (returning whether it did), behind the next block's reads; after(mb) runs once
// block mb's output is complete (VALU work of the caller that the next block's MFMAs follow).
template <typename Emit = NoEmit, typename After = NoAfter>
__device__ __forceinline__ void forward_layer(const float* s_small, const float* w_rows, int layer,
                                              int g, const f4 (&hin)[4][4], f4 (&hout)[4][4],
                                              Emit emit = Emit{}, After after = After{}) {
  f4 bias[4];
  load_bias(s_small, layer, g, bias);
  const float* w = w_rows + layer * kPlane;
  f4 next[4];
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) next[ob] = lds4(w + 16 * ob);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    f4 a[4];
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) a[ob] = next[ob];
    if (mb < 3) {
#pragma unroll
      for (int ob = 0; ob < 4; ++ob) next[ob] = lds4(w + 1088 * (mb + 1) + 16 * ob);
    }
    lds_mfma_fence();
    f4 z[4];
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f4 cin = (ob | j) ? z[c] : (c == 0 ? bias[mb] : zero4());
          z[c] = mfma(a[ob][j], hin[ob][c][j], cin);
        }
        if (emit(mb, 4 * ob + j)) __builtin_amdgcn_sched_barrier(0);
      }
    }
    lds_mfma_fence();  // the next block's reads stay ahead of this block's MFMAs
    tanh_jet4(z, hout[mb]);
    after(mb);
  }
}

// A operands of transposed_block for input block ib: W[16 ob + 4 g + j][16 ib + m] for the 16
// k-steps (ob, j), 4-byte LDS reads from this lane's column base w (272 g + m) in the layer's
// pitch-68 plane.
__device__ __forceinline__ void transposed_operands(const float* w, int ib, float (&a)[16]) {
#pragma unroll
  for (int step = 0; step < 16; ++step) a[step] = w[1088 * (step >> 2) + kWRow * (step & 3) + 16 * ib];
}

// hb[c] = sum_o W[o][16 ib + .] zb[o][c][.] for one input block ib: 64 MFMAs over the k-steps
// (ob, j) in order, from the operands a of
// transposed_operands.
__device__ __forceinline__ void transposed_block(const float (&a)[16], const f4 (&zb)[4][4],
                                                 f4 (&hb)[4]) {
#pragma unroll
  for (int step = 0; step < 16; ++step) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      hb[c] = mfma(a[step], zb[step >> 2][c][step & 3], step ? hb[c] : zero4());
    }
  }
}

// The adjoint through one hidden layer's weights and the tanh jet below it, one input block at
// a time: hbar = W^T zbar for block ib, then the tanh-jet adjoint of that block of the layer
// below, from its output hp, which replaces hp[ib] by the layer below's zbar. Only one block of
// hbar is live at a time. after(ib) runs once block ib's adjoint is done (VALU work of the caller
// for that block); emit(ib, step) may issue LDS writes of block ib after k-step `step` of block
// ib + 1's MFMAs (returning whether it did), behind block ib + 2's operand reads, and block 3's
// writes follow its adjoint.
template <typename After, typename Emit>
__device__ __forceinline__ void adjoint_through(const float* w, const f4 (&zb)[4][4],
                                                f4 (&hp)[4][4], After after, Emit emit) {
  float next[16];
  transposed_operands(w, 0, next);
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) {
    float a[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) a[k] = next[k];
    if (ib < 3) transposed_operands(w, ib + 1, next);
    lds_mfma_fence();
    f4 hb[4];
#pragma unroll
    for (int step = 0; step < 16; ++step) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        hb[c] = mfma(a[step], zb[step >> 2][c][step & 3], step ? hb[c] : zero4());
      }
      if (ib > 0 && emit(ib - 1, step)) __builtin_amdgcn_sched_barrier(0);
    }
    lds_mfma_fence();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float bv = hb[0][r], bj0 = hb[1][r], bj1 = hb[2][r], bl = hb[3][r];
      tanh_jet_adjoint_h(hp[ib][0][r], hp[ib][1][r], hp[ib][2][r], hp[ib][3][r], bv, bj0, bj1, bl);
      hp[ib][0][r] = bv;
      hp[ib][1][r] = bj0;
      hp[ib][2][r] = bj1;
      hp[ib][3][r] = bl;
    }
    after(ib);
  }
#pragma unroll
  for (int step = 0; step < 16; ++step) emit(3, step);
}

// Staging writes of a block's early components spread over the 16 k-steps of a block of MFMAs:
// writes 2 step and 2 step + 1 of stage_early_write after k-step `step` < 12.
__device__ __forceinline__ bool emit_early_pair(const StageBases& sb, int mb, const f4 (&x)[4],
                                                const f4 (&y)[4], int step) {
  if (step >= 12) return false;
  stage_early_write(sb, mb, x, y, 2 * step);
  stage_early_write(sb, mb, x, y, 2 * step + 1);
  return true;
}

// Seed of the fused Poisson training step (kLoss). The loss is the PINN loss
//   mean_interior (lap - f)^2 + w mean_boundary u^2
// (/root/reference/src/fused_hoad/training.py:66-88; with no boundary points, the loss of
// /root/reference/benchmarks/benchmark_training.py:46-48). The kernel already re-runs the
// forward, so it forms the upstream gradients autograd would form for that loss itself:
//   interior points: grad_u = 0, grad_lap = fl(1 / B) (2 r) with r = lap - f;
//   boundary points: grad_u = fl(w / B_b) (2 u), grad_lap = 0.
// Tiles [0, interior_tiles) hold interior points and the rest boundary points, 16 per tile in
// both gradient kernels (boundary_tile, backward_split_kernel). sum r^2 and
// sum u^2 go into columns kLossColumn and kLossColumn + 1 of the slot's partial row. `step` is
// the Adam step counter, advanced here (one lane of workgroup 0) so that the update kernel that
// follows reads a settled value.
struct LossSeed {
  const float* source;     // f[batch]
  const float* boundary;   // boundary coordinates [boundary_count][2]
  int64_t interior_tiles;  // ceil(batch / 64) (backward_kernel) or ceil(batch / 16) (split)
  int64_t boundary_count;
  float inv_batch;         // fl(1 / B)
  float boundary_scale;    // fl(fl(w) / B_b)
  float* step;             // Adam step counter (one float)
};

constexpr int kLossColumn = kParameterCount;  // partial-row columns of sum r^2, sum u_b^2
static_assert(kLossColumn + 1 < kRowStride, "the loss columns must fit in a partial row");

// Per-slot gradient sums of one wave (see backward_kernel).
struct WaveSums {
  f4 dw[3][4];         // hidden dW, rows 16 w + ., in MFMA accumulator layout
  float bh[3];         // hidden bias sums of c^-1 zbar_v (row 16 w + m, see dw_pass)
  float w0x, w0y, b0;  // layer-0 sums, lane = owned neuron
  float wout, bout;    // output-layer sums
  float loss, bloss;   // kLoss: sums of r^2 and u_b^2
};

// A boundary tile of the fused step. Boundary points enter the loss through u alone
// (grad_lap = 0), so the output seed is (vbar', Jbar', Lbar') = (4 gu w_out / c, 0, 0), and the
// tanh-jet adjoint maps (vbar', 0, 0, 0) to (s' vbar', 0, 0, 0): every adjoint component but
// the value one is exactly zero at every layer. The weight-gradient terms reduce to
// zbar_v h_v^T, and the forward's J and L components feed nothing. A boundary tile therefore
// runs the value channel only; the terms it skips are exact zeros.
//
// A boundary tile holds 16 points, shared by the workgroup's 4 waves: wave w owns rows
// 16 w .. 16 w + 15 of every layer, so the forward, dW and W^T zbar products of a layer are 16
// MFMAs each per wave (a 16-point value-channel tile on one wave would be 64 each). Layer
// outputs and adjoints go to the other waves lane to lane through LDS (the register layout of
// forward_split_kernel: register r of block ob holds row 16 ob + 4 g + r at point m), for the
// next product's B operand. dW contracts over the tile's points, which sit on the lane axis, so
// each layer's h_v and the wave's zbar_v are also stored transposed: row R, point 4 s + g at
// column 4 g + s of a 20-float row, so one 16-byte read gives a lane the points of its 4 k-steps.
// Scratch inside the dW staging buffer (floats):
constexpr int kBndPitch = 20;                                   // transposed row, 16 points + pad
constexpr int kBndExchange = 0;                                 // [2][4 waves][64 lanes] f4
constexpr int kBndH = kBndExchange + 2 * kBwdWaves * kWave * 4;  // [3 layers][64 rows][pitch]
constexpr int kBndZ = kBndH + 3 * kHidden * kBndPitch;          // [2][4 waves][16 rows][pitch]
static_assert(kBndZ + 2 * kBwdWaves * 16 * kBndPitch <= kStagePlanes * kPlane,
              "the boundary tile's scratch must fit the dW staging buffer");

// Store this lane's 4 rows row0 + 4 g + r (value at point m) into a transposed buffer.
__device__ __forceinline__ void store_point_columns(float* t, int row0, int g, int m, f4 x) {
  const int col = 4 * (m & 3) + (m >> 2);
#pragma unroll
  for (int r = 0; r < 4; ++r) t[(row0 + 4 * g + r) * kBndPitch + col] = x[r];
}

// Per-neuron point sums of this wave's rows: t[r] is the total of row 16 w + 4 g + r (the same
// in all 16 lanes of row g). Lane (m, g) owns neuron owned_neuron(m, g) =
// 16 (m >> 2) + 4 g + (m & 3) in the slot sums, so it takes t[m & 3] when m >> 2 == w and adds
// nothing otherwise (the other waves own those neurons' rows).
__device__ __forceinline__ float own_row_total(const f4 t, int m, int w) {
  const float lo = (m & 1) ? t[1] : t[0];
  const float hi = (m & 1) ? t[3] : t[2];
  const float v = (m & 2) ? hi : lo;
  return (m >> 2) == w ? v : 0.0f;
}

__device__ __forceinline__ f4 row_totals(const f4 x) {
  f4 t;
#pragma unroll
  for (int r = 0; r < 4; ++r) t[r] = sum_row16(x[r]);
  return t;
}

__device__ __forceinline__ void boundary_tile(const float* s_w, const float* s_small,
                                              float* s_stage, int rows_off, int cols_off, int w,
                                              int g, int m, float x0, float x1, bool active,
                                              float boundary_scale, WaveSums& acc) {
  __syncthreads();  // the previous tile's readers of the staging buffer are done
  f4* xch = reinterpret_cast<f4*>(s_stage + kBndExchange);
  float* ht = s_stage + kBndH;
  float* zt = s_stage + kBndZ;
  const int lane = 16 * g + m;
  int phase = 0;  // alternates the exchange and zbar buffers

  // ---- forward, value channel: layer 0 whole, then this wave's rows of hidden layers 1..3 ----
  f4 h[4];      // v' of all 64 rows of the current layer output
  f4 s_own[3];  // s' of this wave's rows of layer 0 and hidden layers 1, 2
  f4 v_top, s_top;  // hidden layer 3, this wave's rows
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) {
    const Layer0Weights w0 = layer0_weights(s_small, ob, g);
    f4 zv, unused;
#pragma unroll
    for (int r = 0; r < 4; ++r) zv[r] = layer0_zv(w0, r, x0, x1);
    tanh_scaled4(zv, h[ob], unused);
  }
  {
    // this wave's block again (h[w] would need a dynamic register index)
    const Layer0Weights w0 = layer0_weights(s_small, w, g);
    f4 zv, v;
#pragma unroll
    for (int r = 0; r < 4; ++r) zv[r] = layer0_zv(w0, r, x0, x1);
    tanh_scaled4(zv, v, s_own[0]);
    store_point_columns(ht, 16 * w, g, m, v);
  }
#pragma unroll
  for (int l = 0; l < 3; ++l) {
    const f4 b = lds4(s_small + kSmallBh + l * kHidden + 16 * w + 4 * g);
    const float* wrow = s_w + l * kPlane + opaque(rows_off) + 1088 * w;  // W[16 w + m][.]
    f4 z;
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      const f4 a = lds4(wrow + 16 * ob);
#pragma unroll
      for (int j = 0; j < 4; ++j) z = mfma(a[j], h[ob][j], (ob | j) ? z : b);
    }
    f4 v, sl;
    tanh_scaled4(z, v, sl);
    if (l < 2) {
      s_own[l + 1] = sl;
      store_point_columns(ht + (l + 1) * kHidden * kBndPitch, 16 * w, g, m, v);
    } else {
      v_top = v;
      s_top = sl;
    }
    xch[(phase * kBwdWaves + w) * kWave + lane] = v;
    __syncthreads();
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) h[ob] = xch[(phase * kBwdWaves + ob) * kWave + lane];
    phase ^= 1;
  }

  // ---- u = w_out . v + b_out over all 64 rows, the seed gu = fl(w / B_b) (2 u) ----
  float out = 0.0f;
#pragma unroll
  for (int ob = 0; ob < 4; ++ob) {
    const f4 wo = lds4(s_small + kSmallWoutV + 16 * ob + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r) out = __builtin_fmaf(wo[r], h[ob][r], out);
  }
  out = sum_lane_groups(out);
  const float u = active ? out + s_small[kSmallBout] : 0.0f;
  const float gu = boundary_scale * (2.0f * u);
  if (w == 0) {  // the 4 waves share the tile's points: one of them adds the point sums
    acc.bloss += sum_row16(u * u);
    acc.bout += sum_row16(gu);
  }
  const float gu_c = gu * (4.0f / kC);
  acc.wout += own_row_total(row_totals(gu_c * v_top), m, w);
  const f4 wv = lds4(s_small + kSmallWoutV + 16 * w + 4 * g);
  f4 zb = s_top * (gu * wv);  // hidden layer 3's zbar_v' = s' vbar', this wave's rows

  // ---- hidden layers 3, 2, 1: dW, the bias sum, hbar = W^T zbar, the next zbar ----
#pragma unroll
  for (int l = 2; l >= 0; --l) {
    float* ztw = zt + (phase * kBwdWaves + w) * 16 * kBndPitch;
    store_point_columns(ztw, 0, g, m, zb);
    xch[(phase * kBwdWaves + w) * kWave + lane] = zb;
    __syncthreads();
    {
      // dW[16 w + ., 16 nb + .] += sum over the 16 points of zbar h_prev^T: A = zbar of row
      // 16 w + m, B = h_prev of row 16 nb + m, k-step s = points 4 s + g.
      const f4 a = lds4(ztw + m * kBndPitch + 4 * g);
      const float* hrow = ht + l * kHidden * kBndPitch + m * kBndPitch + 4 * g;
      f4 bt[4];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) bt[nb] = lds4(hrow + 16 * nb * kBndPitch);
      float bsum = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        bsum += a[k];
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc.dw[l][nb] = mfma(a[k], bt[nb][k], acc.dw[l][nb]);
      }
      acc.bh[l] += sum_lane_groups(bsum);
    }
    f4 hb;
    {
      // hbar of this wave's rows of the layer below: sum over the 64 rows o of
      // W[o][16 w + m] zbar[o].
      const float* wt = s_w + l * kPlane + opaque(cols_off) + 16 * w;
#pragma unroll
      for (int ob = 0; ob < 4; ++ob) {
        const f4 zo = xch[(phase * kBwdWaves + ob) * kWave + lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          hb = mfma(wt[1088 * ob + kWRow * j], zo[j], (ob | j) ? hb : zero4());
        }
      }
    }
    phase ^= 1;
    zb = s_own[l] * hb;  // zbar_v' of the layer below (l = 0: layer 0's bv)
  }

  // ---- layer 0: dW0[o][d] = 2 sum_p bv (c x_d / 2) (the row takes the 2), db0 = c sum_p bv ----
  const float cx0 = kHalfC * x0, cx1 = kHalfC * x1;
  acc.w0x += own_row_total(row_totals(zb * cx0), m, w);
  acc.w0y += own_row_total(row_totals(zb * cx1), m, w);
  acc.b0 += own_row_total(row_totals(zb), m, w);
}

// Per-point inputs of one gradient-kernel tile for this lane: coordinates and, for interior
// points, the upstream gradients (gu, gl) or, with kLoss, the source f (in a). Boundary tiles
// (kLoss, tile >= seed.interior_tiles) take boundary coordinates. Inactive lanes get zeros.
struct TileInputs {
  float x0, x1, a, b;
};

template <bool kLoss, bool kRest = false>
__device__ __forceinline__ TileInputs load_tile_inputs(const float* __restrict__ coordinates,
                                                       const float* __restrict__ grad_output,
                                                       const float* __restrict__ grad_laplacian,
                                                       int64_t batch, int64_t whole,
                                                       const LossSeed& seed, int64_t tile, int w,
                                                       int m) {
  TileInputs in{0.f, 0.f, 0.f, 0.f};
  if (kLoss && tile >= seed.interior_tiles) {  // 16-point boundary tile, shared by the waves
    const int64_t point = (tile - seed.interior_tiles) * kTile + m;
    if (point < seed.boundary_count) {
      in.x0 = seed.boundary[2 * point];
      in.x1 = seed.boundary[2 * point + 1];
    }
    return in;
  }
  // 64-point tiles below `whole`, then (kRest) 16-point tiles shared by the waves (split_tile).
  const int64_t point = !kRest || tile < whole ? tile * kBwdTile + kTile * w + m
                                               : whole * kBwdTile + (tile - whole) * kTile + m;
  if (point < batch) {
    in.x0 = coordinates[2 * point];
    in.x1 = coordinates[2 * point + 1];
    if (kLoss) {
      in.a = seed.source[point];
    } else {
      in.a = grad_output ? grad_output[point] : 0.0f;  // a null upstream gradient is zero
      in.b = grad_laplacian ? grad_laplacian[point] : 0.0f;
    }
  }
  return in;
}

// Force delivery of prefetched inputs at this point (an opaque use of each register).
__device__ __forceinline__ void deliver(TileInputs& in) {
  in.x0 = opaque(in.x0);
  in.x1 = opaque(in.x1);
  in.a = opaque(in.a);
  in.b = opaque(in.b);
}

constexpr int kSplitBwdMaxTiles = 768;  // backward_split_kernel up to 768 16-point tiles
constexpr int kTPlane = 64 * kWRow;     // floats of one transposed 64-row layer (h)
constexpr int kTWave = 16 * kWRow;      // floats of one wave's transposed zbar

// Store this lane's 4 rows (rows0 + 4 g + r) x 4 components at point m into a transposed
// buffer t[row][68]: component c of point p = 4 s + g' at t[row * 68 + 16 c + 4 g' + s].
__device__ __forceinline__ void store_transposed(float* t, int rows0, int g, int m,
                                                 const f4 (&x)[4]) {
  const int col = 4 * (m & 3) + (m >> 2);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int c = 0; c < 4; ++c) t[(rows0 + 4 * g + r) * kWRow + 16 * c + col] = x[c][r];
  }
}

// Scratch of one 16-point tile whose rows are split over the workgroup's 4 waves.
struct SplitScratch {
  float* ht;                       // [3][kTPlane]: h of layers 0..2, transposed
  f4 (*x)[kSplitWaves][4][kWave];  // [2 buffers]: lane-major exchange
  float (*zt)[kTWave];             // [4 waves]: this wave's zbar, transposed
  float (*gx)[2][kTile];           // [4 waves]: partial coordinate gradients
};
constexpr int kSplitScratchFloats = 3 * kTPlane + 2 * kSplitWaves * 4 * kWave * 4 +
                                    kSplitWaves * kTWave + kSplitWaves * 2 * kTile;

// Per-lane point sums of split_tile: bias sums go to the caller's array (row 16 w + m, as in
// dw_pass); these are of row 16 w + 4 g + (m & 3) (w0x, w0y, b0, wout), or the same in every
// lane of a wave (bout, loss, bloss).
struct SplitSums {
  float w0x, w0y, b0, wout, bout, loss, bloss;
};

// One 16-point tile, all 4 waves: wave w owns rows 16 w .. 16 w + 15 of every layer (64 MFMAs
// per layer for the forward re-run, dW and W^T zbar). Layer outputs and adjoints go to the
// other waves lane to lane through LDS (`sc.x`, the register layout of forward_split_kernel),
// and each layer's h (all 64 rows) and the wave's zbar are also stored transposed,
// [row][c][4 g + s] for point 4 s + g at pitch 68, so dW contracts over the tile's points with
// 16-byte reads. dW and the bias sums accumulate into `dw` / `bias` (the layout of
// backward_kernel's); grad_coordinates of interior points are written here. `rows_off` and
// `cols_off` are this wave's lane offsets W[16 w + m][.] and W[.][16 w + m]; t_read = 68 m + 4 g.
template <bool kLoss>
__device__ __forceinline__ void split_tile(const float* s_w, const float* s_small,
                                           const SplitScratch& sc, int& phase, int w, int g, int m,
                                           int rows_off, int cols_off, int t_read, float x0,
                                           float x1, float gu, float gl, float f, bool active,
                                           bool on_boundary, int64_t point,
                                           float* __restrict__ grad_coordinates,
                                           const LossSeed& seed, f4 (&dw)[3][4], float (&bias)[3],
                                           SplitSums& sums) {
  const int lane = 16 * g + m;
  // ---- forward re-run: all 64 rows of layer 0, then this wave's rows of layers 1..3 ----
  f4 h[4][4];
  layer0_forward(s_small, g, x0, x1, h);
  {
    f4 own[4];  // this wave's block again (h[w] would need a dynamic register index)
    layer0_block(s_small, w, g, x0, x1, own);
    store_transposed(sc.ht, 16 * w, g, m, own);
  }
  f4 z[3][4];  // this wave's pre-activations of hidden layers 1..3
  f4 mine[4];  // this wave's rows of the current layer output
#pragma unroll
  for (int layer = 0; layer < 3; ++layer) {
    const f4 b = lds4(s_small + kSmallBh + layer * kHidden + 16 * w + 4 * g);
    const float* wrow = s_w + layer * kPlane + opaque(rows_off);
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
      const f4 a = lds4(wrow + 16 * ob);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f4 cin = (ob | j) ? z[layer][c] : (c == 0 ? b : zero4());
          z[layer][c] = mfma(a[j], h[ob][c][j], cin);
        }
      }
    }
    tanh_jet4(z[layer], mine);
    f4 (*xb)[4][kWave] = sc.x[phase];
    phase ^= 1;
#pragma unroll
    for (int c = 0; c < 4; ++c) xb[w][c][lane] = mine[c];
    if (layer < 2) store_transposed(sc.ht + (layer + 1) * kTPlane, 16 * w, g, m, mine);
    __syncthreads();
#pragma unroll
    for (int ob = 0; ob < 4; ++ob) {
#pragma unroll
      for (int c = 0; c < 4; ++c) h[ob][c] = xb[ob][c][lane];  // this wave's block included
    }
  }

  if (kLoss) {
    // u (boundary) or lap (interior) over all 64 rows, in backward_kernel's order.
    float out = 0.0f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const f4 wo = lds4(s_small + (on_boundary ? kSmallWoutV : kSmallWoutL) + 16 * mb + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        out = __builtin_fmaf(wo[r], on_boundary ? h[mb][0][r] : h[mb][3][r], out);
      }
    }
    out = sum_lane_groups(out);
    // u (boundary) or the residual lap - f (interior); both sums are updated with a select, so
    // that `sums` stays in registers (a branch per field made the compiler address it).
    const float e = active ? (on_boundary ? out + s_small[kSmallBout] : out - f) : 0.0f;
    if (on_boundary) {
      gu = seed.boundary_scale * (2.0f * e);
    } else {
      gl = seed.inv_batch * (2.0f * e);
    }
    const float sq = sum_row16(e * e);
    sums.bloss += on_boundary ? sq : 0.0f;
    sums.loss += on_boundary ? 0.0f : sq;
  }

  // ---- output layer: this wave's rows of the seed and of dw_out ----
  f4 hb[4];
  {
    const float gu_c = gu * (4.0f / kC);
    const float gl_l = gl * (4.0f / kLambda);
    const f4 wv = lds4(s_small + kSmallWoutV + 16 * w + 4 * g);
    const f4 wl = lds4(s_small + kSmallWoutL + 16 * w + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float total = sum_row16(__builtin_fmaf(gu_c, mine[0][r], gl_l * mine[3][r]));
      sums.wout = (m & 3) == r ? sums.wout + total : sums.wout;
      hb[0][r] = gu * wv[r];
      hb[1][r] = 0.0f;
      hb[2][r] = 0.0f;
      hb[3][r] = gl * wl[r];
    }
    sums.bout += sum_row16(gu);
  }

  // ---- hidden layers 3, 2, 1 ----
#pragma unroll
  for (int layer = 2; layer >= 0; --layer) {
    // zbar of this wave's rows (tanh-jet adjoint, lane-local)
    f4 zb[4];
    f4 v4, s4;
    tanh_scaled4(z[layer][0], v4, s4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = v4[r], s = s4[r];
      float bv = hb[0][r], bj0 = hb[1][r], bj1 = hb[2][r], bl = hb[3][r];
      tanh_jet_adjoint_vs(v, s, z[layer][1][r], z[layer][2][r], z[layer][3][r], bv, bj0, bj1,
                          bl);
      zb[0][r] = bv;
      zb[1][r] = bj0;
      zb[2][r] = bj1;
      zb[3][r] = bl;
    }
    f4 (*xb)[4][kWave] = sc.x[phase];
    phase ^= 1;
#pragma unroll
    for (int c = 0; c < 4; ++c) xb[w][c][lane] = zb[c];
    float* zt = sc.zt[w];
    store_transposed(zt, 0, g, m, zb);
    __syncthreads();
    // dW[16 w + ., 16 nb + .] += sum over (c, points) of zbar h_prev^T; the A reads of
    // component 0 also give the bias sum of row 16 w + m.
    {
      const float* ht = sc.ht + layer * kTPlane + opaque(t_read);
      const float* za = zt + opaque(t_read);
      float bsum = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f4 a = lds4(za + 16 * c);
        f4 bt[4];
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) bt[nb] = lds4(ht + 16 * kWRow * nb + 16 * c);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          if (c == 0) bsum += a[s];
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) dw[layer][nb] = mfma(a[s], bt[nb][s], dw[layer][nb]);
        }
      }
      bias[layer] += sum_lane_groups(bsum);
    }
    // hbar of this wave's rows of the layer below: sum over all 64 rows o of
    // W[o][16 w + .] zbar[o].
    {
      const float* wt = s_w + layer * kPlane + opaque(cols_off);
#pragma unroll
      for (int ob = 0; ob < 4; ++ob) {
        f4 zo[4];  // zbar of rows 16 ob .. 16 ob + 15 (this wave's block included)
#pragma unroll
        for (int c = 0; c < 4; ++c) zo[c] = xb[ob][c][lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a = wt[1088 * ob + kWRow * j];
#pragma unroll
          for (int c = 0; c < 4; ++c) hb[c] = mfma(a, zo[c][j], (ob | j) ? hb[c] : zero4());
        }
      }
    }
  }

  // ---- layer 0 for this wave's rows: dW0, db0 and this wave's part of grad_x ----
  {
    const Layer0Weights w0 = layer0_weights(s_small, w, g);
    const float cx0 = kHalfC * x0, cx1 = kHalfC * x1;
    float gx0 = 0.f, gx1 = 0.f;
    f4 zv4, v4, s4;
#pragma unroll
    for (int r = 0; r < 4; ++r) zv4[r] = layer0_zv(w0, r, x0, x1);
    tanh_scaled4(zv4, v4, s4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = v4[r], s = s4[r];
      float bv = hb[0][r], bj0 = hb[1][r], bj1 = hb[2][r], bl = hb[3][r];
      tanh_jet_adjoint_vs(v, s, w0.wx[r], w0.wy[r], 0.0f, bv, bj0, bj1, bl);
      gx0 = __builtin_fmaf(w0.cwx[r], bv, gx0);
      gx1 = __builtin_fmaf(w0.cwy[r], bv, gx1);
      const float t0 = sum_row16(__builtin_fmaf(bv, cx0, bj0));
      const float t1 = sum_row16(__builtin_fmaf(bv, cx1, bj1));
      const float tb = sum_row16(bv);
      sums.w0x = (m & 3) == r ? sums.w0x + t0 : sums.w0x;
      sums.w0y = (m & 3) == r ? sums.w0y + t1 : sums.w0y;
      sums.b0 = (m & 3) == r ? sums.b0 + tb : sums.b0;
    }
    gx0 = sum_lane_groups(gx0);
    gx1 = sum_lane_groups(gx1);
    if (g == 0) {
      sc.gx[w][0][m] = gx0;
      sc.gx[w][1][m] = gx1;
    }
    __syncthreads();
    if (w == 0 && g == 0 && active && grad_coordinates != nullptr && !on_boundary) {
      grad_coordinates[2 * point] = ((sc.gx[0][0][m] + sc.gx[1][0][m]) + sc.gx[2][0][m]) + sc.gx[3][0][m];
      grad_coordinates[2 * point + 1] = ((sc.gx[0][1][m] + sc.gx[1][1][m]) + sc.gx[2][1][m]) + sc.gx[3][1][m];
    }
  }
}

// Phase clock of backward_kernel, compiled only into a measurement build (-DFHOAD_PHASE_CLOCK;
// the library build reads no clock and every mark below compiles to nothing). Each wave adds
// the shader-clock cycles (s_memtime) it spends in each phase of its tiles to its row of
// g_phase_clock and counts its tiles; fhoad_phase_clock_read copies the table out. A clock
// read waits for the wave's outstanding LDS and scalar loads, so the measured kernel runs
// somewhat slower than the library's.
enum ClockField : int {
  kClockStage,          // kernel start to the end of the parameter staging
  kClockForward,        // a tile's start: layer 0 and hidden layers 1, 2 (the forward re-run)
  kClockLayer3,         // hidden layer 3's forward, the loss and output seed, zbar3's staging
  kClockDw3,            // dW3 (three staged passes)
  kClockAdjoint3,       // W3^T zbar3 into layer 2's adjoint
  kClockDw2,            // dW2
  kClockAdjoint2,       // W2^T zbar2 into layer 1's adjoint, layer 0 rebuilt
  kClockDw1,            // dW1
  kClockLayer0,         // W1^T zbar1, layer 0's adjoint, coordinate gradients
  kClockRest,           // 16-point split tiles past the last whole round
  kClockBoundary,       // boundary tiles of the fused step
  kClockPartials,       // the slot's partial row
  kClockTiles,          // count of 64-point tiles
  kClockBoundaryTiles,  // count of boundary tiles
  kClockWallStart,      // s_memrealtime (100 MHz) at the kernel's start
  kClockWallEnd,        // s_memrealtime after the partial row's stores are issued
  kClockFields
};
constexpr int kClockWorkgroups = 1024;  // rows kept: workgroups 0 .. 1023

#ifdef FHOAD_PHASE_CLOCK
__device__ unsigned long long g_phase_clock[kClockWorkgroups][kBwdWaves][kClockFields];

struct PhaseClock {
  unsigned long long last, fields[kClockFields];
  __device__ __forceinline__ PhaseClock() {
#pragma unroll
    for (int i = 0; i < kClockFields; ++i) fields[i] = 0;
    fields[kClockWallStart] = wall_clock64();
    last = clock64();
  }
  __device__ __forceinline__ void mark(ClockField field) {
    const unsigned long long now = clock64();
    fields[field] += now - last;
    last = now;
  }
  __device__ __forceinline__ void count(ClockField field) { fields[field] += 1; }
  __device__ __forceinline__ void store(int w) {
    fields[kClockWallEnd] = wall_clock64();
    if ((threadIdx.x & (kWave - 1)) == 0 && blockIdx.x < kClockWorkgroups) {
#pragma unroll
      for (int i = 0; i < kClockFields; ++i) g_phase_clock[blockIdx.x][w][i] = fields[i];
    }
  }
};
#else
struct PhaseClock {
  __device__ __forceinline__ void mark(ClockField) {}
  __device__ __forceinline__ void count(ClockField) {}
  __device__ __forceinline__ void store(int) {}
};
#endif

// The outputs h1, h2, h3 of the hidden layers stay in registers through the walk back (each
// layer's zbar replaces its h in place, and hbar is live one 16-row block at a time), so no
// layer is parked in memory.
//
// kLoss: grad_output and grad_laplacian are unused and the seed comes from `seed` (above);
// grad_coordinates may be null.
// kSaved (backward call only): interior tiles read h1, h2, h3 from `saved`, written by the
// saving forward (saved_index; saved_tiles 16-point tiles), instead of re-running the forward.
// A wave whose 16-point tile lies past the batch takes zeros: its upstream gradients are zero,
// so every product with its h is zero either way. Split tiles past the last whole round still
// re-run the forward.
template <bool kLoss, bool kRest, bool kSaved>
__global__ void __launch_bounds__(kBwdWaves * kWave, 1)
backward_kernel(const float* __restrict__ coordinates, const float* __restrict__ params,
                const float* __restrict__ grad_output, const float* __restrict__ grad_laplacian,
                float* __restrict__ grad_coordinates, float* __restrict__ partials,
                int64_t batch, int64_t whole, int64_t tiles, int slots, LossSeed seed,
                const f4* __restrict__ saved, int64_t saved_tiles) {
  static_assert(!(kLoss && kSaved), "the fused step computes its forward once; nothing to read");
  constexpr int kStageFloats = kRest && kSplitScratchFloats > kStagePlanes * kPlane
                                   ? kSplitScratchFloats
                                   : kStagePlanes * kPlane;
  __shared__ __attribute__((aligned(16))) float s_w[3 * kPlane];
  __shared__ __attribute__((aligned(16))) float s_small[kSmallFloats];
  __shared__ __attribute__((aligned(16))) float s_stage[kStageFloats];
  __shared__ float s_red[3][kBwdWaves];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int m = lane & 15;
  const int g = lane >> 4;
  PhaseClock clock;
  // The first slot's first tile inputs are read before the staging, which hides their latency.
  TileInputs next{0.f, 0.f, 0.f, 0.f};
  if (static_cast<int>(blockIdx.x) < slots) {
    next = load_tile_inputs<kLoss, kRest>(coordinates, grad_output, grad_laplacian, batch, whole, seed,
                                   blockIdx.x, w, m);
  }
  // kLoss: the Adam step count is read with the staging loads and advanced after the barrier
  // (an increment in place waited for its load before wave 0 issued any staging load).
  const float step_count = kLoss ? seed.step[0] : 0.0f;
  stage_parameters<kBwdWaves * kWave>(params, s_w, s_small, threadIdx.x);
  __syncthreads();
  if (kLoss && blockIdx.x == 0 && threadIdx.x == 0) seed.step[0] = step_count + 1.0f;
  clock.mark(kClockStage);

  // Lane offsets into the LDS arrays. Each use forms its base from an opaque copy: the arrays
  // span more than the 64 KB reach of a DS offset, and hoisted bases would be spilled.
  const int rows_off = lane_rows(m, g);
  const int cols_off = lane_cols(m, g);
  const int stage_write_off = cols_off + 16 * w;    // staging writes: point 16 w + m
  const int stage_a_off = rows_off + 16 * kWRow * w;  // A operand reads: this wave's rows
  auto stage_bases = [&]() {
    const int wo = opaque(stage_write_off), ao = opaque(stage_a_off), ro = opaque(rows_off);
    return StageBases{s_stage + wo, s_stage + 3 * kPlane + wo, s_stage + ao,
                      s_stage + 3 * kPlane + ro};
  };

  for (int slot = blockIdx.x; slot < slots; slot += gridDim.x) {
    WaveSums acc;
#pragma unroll
    for (int l = 0; l < 3; ++l) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) acc.dw[l][nb] = zero4();
      acc.bh[l] = 0.f;
    }
    acc.w0x = acc.w0y = acc.b0 = acc.wout = acc.bout = acc.loss = acc.bloss = 0.f;

    // Per-point inputs are read one tile ahead and delivered mid-tile (deliver), so no tile
    // starts with a wait on global memory: with one wave per SIMD nothing would hide it. The
    // delivery sits before the tile's own stores, which a wait at the next tile's head would
    // also have to wait for (they are behind branches, so the compiler cannot count them).
    if (slot != static_cast<int>(blockIdx.x)) {
      next = load_tile_inputs<kLoss, kRest>(coordinates, grad_output, grad_laplacian, batch, whole, seed, slot,
                                     w, m);
    }
    deliver(next);
    // A slot's interior tiles come before its boundary tiles (kLoss), so two loops run them in
    // the same order as one would. One loop with both kinds of tile cost about 100 register
    // copies a tile, where the two paths' accumulators met at the loop's back edge.
    int64_t tile = slot;
    const int64_t interior_end = kLoss ? std::min<int64_t>(tiles, seed.interior_tiles) : tiles;
    const int64_t loop_end = kRest ? whole : interior_end;
    // Hidden-layer outputs of the current tile. With kSaved each layer of the next tile is read
    // where this tile's copy dies in the walk back (layer 3 after W3^T zbar3, layer 2 after
    // W2^T zbar2, layer 1 at the end), so the reads spread over the tile: read at each tile's
    // start, the waves of all CUs asked for their 48 KB at once and waited out that burst.
    // (Reading a slot's first tile before the weight staging measured no faster.)
    f4 h1[4][4], h2[4][4], h3[4][4];
    if constexpr (kSaved) {
      if (tile < loop_end) {
        const int64_t saved_tile = kBwdWaves * tile + w;
        load_saved_layer(saved, saved_tile, saved_tiles, 2, lane, h3);
        load_saved_layer(saved, saved_tile, saved_tiles, 1, lane, h2);
        load_saved_layer(saved, saved_tile, saved_tiles, 0, lane, h1);
      }
    }
    for (; tile < loop_end; tile += slots) {
      const bool has_next = tile + slots < loop_end;
      const int64_t next_saved_tile = kBwdWaves * (tile + slots) + w;
      keep_lds_reads_in_loop();
      const int m_pick = opaque(m);  // row_reduce_scatter16's lane masks stay inside the tile
      const TileInputs in = next;
      if (tile + slots < tiles) {
        next = load_tile_inputs<kLoss, kRest>(coordinates, grad_output, grad_laplacian, batch, whole, seed,
                                       tile + slots, w, m);
      }
      const float x0 = in.x0, x1 = in.x1;
      const int64_t point = tile * kBwdTile + kTile * w + m;
      const bool active = point < batch;
      float gu = kLoss ? 0.f : in.a, gl = kLoss ? 0.f : in.b;
      const float f = kLoss ? in.a : 0.f;

      // ---- 1. forward recompute (kSaved: read ahead, above and in the walk back) ----
      // h2 is dW3's h_prev: its early components go to the staging planes between hidden layer
      // 3's MFMAs, once every wave is done with the previous tile's planes.
      if constexpr (!kSaved) {
        {
          f4 h0[4][4];
          layer0_forward(s_small, g, x0, x1, h0);
          forward_layer(s_small, s_w + opaque(rows_off), 0, g, h0, h1);
        }
        forward_layer(s_small, s_w + opaque(rows_off), 1, g, h1, h2);
      }
      clock.mark(kClockForward);
      __syncthreads();  // the previous tile's readers of the staging planes are done
      const StageBases sb3 = stage_bases();
      auto stage_h2 = [&](int mb, int step) {
        if (step >= 12) return false;
        const int e = step >> 2, r = step & 3;
        sb3.wh[e * kPlane + kWRow * (16 * mb + r)] = h2[mb][early_component(e)][r];
        return true;
      };
      auto stage_zbar3 = [&](int mb, int i) {  // write i < 12 of zbar3's early components
        sb3.wz[(i >> 2) * kPlane + kWRow * (16 * mb + (i & 3))] = h3[mb][early_component(i >> 2)][i & 3];
      };

      // ---- 2. output layer: w_out / b_out gradients, and hidden layer 3's adjoint ----
      // In the scaled jet u = (4 w_out / c) . v' + b_out and lap = (4 w_out / lambda) . L', so
      // dw_out = sum_p (4 gu / c) v' + (4 gl / lambda) L' and the seeds are
      // vbar' = 4 gu w_out / c, Lbar' = 4 gl w_out / lambda, Jbar' = 0. The point sums stay in
      // registers (row_reduce_scatter16). With kLoss, gu = 0 on interior points: the value seed
      // and the u terms are dropped (their products with zero). h3 becomes zbar3 in place, block
      // by block: in the backward call, whose upstream gradients are inputs, as soon as hidden
      // layer 3's block is done (its staging writes then drain behind the next block's MFMAs);
      // in the fused step after the loss, which needs all of h3.
      float wout_terms[16];
      auto seed_block = [&](int mb) {
        const float gu_c = gu * (4.0f / kC);
        const float gl_l = gl * (4.0f / kLambda);
        const f4 wv = lds4(s_small + kSmallWoutV + 16 * mb + 4 * g);
        const f4 wl = lds4(s_small + kSmallWoutL + 16 * mb + 4 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          wout_terms[4 * mb + r] = kLoss ? gl_l * h3[mb][3][r]
                                         : __builtin_fmaf(gu_c, h3[mb][0][r], gl_l * h3[mb][3][r]);
          float bv = kLoss ? 0.0f : gu * wv[r], bj0, bj1, bl = gl * wl[r];
          tanh_jet_adjoint_h_seed<kLoss>(h3[mb][0][r], h3[mb][1][r], h3[mb][2][r], h3[mb][3][r],
                                         bv, bj0, bj1, bl);
          h3[mb][0][r] = bv;
          h3[mb][1][r] = bj0;
          h3[mb][2][r] = bj1;
          h3[mb][3][r] = bl;
        }
      };
      constexpr bool kSeedInLayer3 = !kLoss && !kSaved;
      if constexpr (kSeedInLayer3) {
        forward_layer(
            s_small, s_w + opaque(rows_off), 2, g, h2, h3,
            [&](int mb, int step) {
              const bool wrote = stage_h2(mb, step);
              if (mb > 0 && step < 12) stage_zbar3(mb - 1, step);
              return wrote || (mb > 0 && step < 12);
            },
            seed_block);
#pragma unroll
        for (int i = 0; i < 12; ++i) stage_zbar3(3, i);
      } else {
        if constexpr (!kSaved) {
          forward_layer(s_small, s_w + opaque(rows_off), 2, g, h2, h3, stage_h2);
        } else {
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
            for (int step = 0; step < 12; ++step) stage_h2(mb, step);
          }
        }
        if (kLoss) {
          // lap = w_out . L in the forward kernel's order, then the seed.
          float out = 0.0f;
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) {
            const f4 wo = lds4(s_small + kSmallWoutL + 16 * mb + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; ++r) out = __builtin_fmaf(wo[r], h3[mb][3][r], out);
          }
          out = sum_lane_groups(out);
          const float res = active ? out - f : 0.0f;
          gl = seed.inv_batch * (2.0f * res);
          acc.loss += sum_row16(res * res);
        }
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          seed_block(mb);
#pragma unroll
          for (int i = 0; i < 12; ++i) stage_zbar3(mb, i);
        }
      }
      acc.wout += row_reduce_scatter16(wout_terms, m_pick);
      if (!kLoss) acc.bout += sum_row16(gu);
      clock.mark(kClockLayer3);

      // ---- 3. hidden layer 3: dW3 from (zbar3, h2), then W3^T zbar3 into layer 2's adjoint ----
      // The adjoint's blocks of zbar2 and h1 (dW2's operands) are staged behind the MFMAs of the
      // next block.
      staged_dw(sb3, {h3[0][kLateComponent], h3[1][kLateComponent], h3[2][kLateComponent], h3[3][kLateComponent]},
                {h2[0][kLateComponent], h2[1][kLateComponent], h2[2][kLateComponent], h2[3][kLateComponent]},
                acc.dw[2], acc.bh[2]);
      clock.mark(kClockDw3);
      __syncthreads();  // every wave is done with the staged planes
      {
        const StageBases sb = stage_bases();
        adjoint_through(s_w + opaque(cols_off) + 2 * kPlane, h3, h2, [](int) {},
                        [&](int ib, int step) { return emit_early_pair(sb, ib, h2[ib], h1[ib], step); });
      }
      if constexpr (kSaved) {
        if (has_next) load_saved_layer(saved, next_saved_tile, saved_tiles, 2, lane, h3);
      }
      clock.mark(kClockAdjoint3);

      // ---- 4. hidden layer 2: dW2 from (zbar2, h1), then W2^T zbar2 into layer 1's adjoint ----
      // Layer 0's output h0 (dW1's h_prev) is rebuilt block by block from its closed form
      // z' = (c (W0 x + b0), 2 W0[:,0], 2 W0[:,1], 0), keeping its (v', s') for layer 0's own
      // adjoint; the blocks of zbar1 and h0 are staged behind the next block's MFMAs.
      f4 v0[4], s0[4], h0[4][4];
      {
        const StageBases sb = stage_bases();
        staged_dw(sb, {h2[0][kLateComponent], h2[1][kLateComponent], h2[2][kLateComponent], h2[3][kLateComponent]},
                  {h1[0][kLateComponent], h1[1][kLateComponent], h1[2][kLateComponent], h1[3][kLateComponent]},
                  acc.dw[1], acc.bh[1]);
        clock.mark(kClockDw2);
        deliver(next);  // the next tile's inputs, before this tile's stores
        __syncthreads();  // every wave is done with the staged planes
        adjoint_through(
            s_w + opaque(cols_off) + kPlane, h2, h1,
            [&](int ib) {
              const Layer0Weights w0 = layer0_weights(s_small, ib, g);
              f4 zv;
#pragma unroll
              for (int r = 0; r < 4; ++r) zv[r] = layer0_zv(w0, r, x0, x1);
              tanh_scaled4(zv, v0[ib], s0[ib]);
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                h0[ib][0][r] = v0[ib][r];
                h0[ib][1][r] = s0[ib][r] * w0.wx[r];
                h0[ib][2][r] = s0[ib][r] * w0.wy[r];
                h0[ib][3][r] = s0[ib][r] * (v0[ib][r] * w0.q[r]);
              }
            },
            [&](int ib, int step) { return emit_early_pair(sb, ib, h1[ib], h0[ib], step); });
      }
      if constexpr (kSaved) {
        if (has_next) load_saved_layer(saved, next_saved_tile, saved_tiles, 1, lane, h2);
      }
      clock.mark(kClockAdjoint2);

      // ---- 5. hidden layer 1: dW1 from (zbar1, h0) ----
      staged_dw(stage_bases(),
                {h1[0][kLateComponent], h1[1][kLateComponent], h1[2][kLateComponent], h1[3][kLateComponent]},
                {h0[0][kLateComponent], h0[1][kLateComponent], h0[2][kLateComponent], h0[3][kLateComponent]},
                acc.dw[0], acc.bh[0]);
      clock.mark(kClockDw1);

      // ---- 6. W1^T zbar1, one block at a time, into layer 0 in closed form ----
      // bv is the adjoint of z'_v = c z_v and bj_d that of z'_Jd = 2 W0[:, d], so
      // grad_x = (c W0)^T bv, dW0[o][d] = sum_p bv (c x_d) + 2 bj_d = 2 sum_p (bv (c x_d / 2) + bj_d)
      // (the row takes the 2), db0 = c sum_p bv.
      {
        float gx0 = 0.f, gx1 = 0.f, tx[16], ty[16], tb[16];
        const float cx0 = kHalfC * x0, cx1 = kHalfC * x1;
        const float* w_t = s_w + opaque(cols_off);
        float next_a[16];
        transposed_operands(w_t, 0, next_a);
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) {
          float a[16];
#pragma unroll
          for (int k = 0; k < 16; ++k) a[k] = next_a[k];
          if (ib < 3) transposed_operands(w_t, ib + 1, next_a);
          lds_mfma_fence();
          f4 hb[4];
          transposed_block(a, h1, hb);
          lds_mfma_fence();
          const Layer0Weights w0 = layer0_weights(s_small, ib, g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float bv = hb[0][r], bj0 = hb[1][r], bj1 = hb[2][r], bl = hb[3][r];
            tanh_jet_adjoint_layer0(v0[ib][r], s0[ib][r], w0.wx[r], w0.wy[r], w0.q[r], bv, bj0,
                                    bj1, bl);
            gx0 = __builtin_fmaf(w0.cwx[r], bv, gx0);
            gx1 = __builtin_fmaf(w0.cwy[r], bv, gx1);
            tx[4 * ib + r] = __builtin_fmaf(bv, cx0, bj0);  // dW0[o][0] / 2
            ty[4 * ib + r] = __builtin_fmaf(bv, cx1, bj1);  // dW0[o][1] / 2
            tb[4 * ib + r] = bv;                            // db0[o] / c
          }
        }
        acc.w0x += row_reduce_scatter16(tx, m_pick);
        acc.w0y += row_reduce_scatter16(ty, m_pick);
        acc.b0 += row_reduce_scatter16(tb, m_pick);
        if constexpr (kSaved) {
          if (has_next) load_saved_layer(saved, next_saved_tile, saved_tiles, 0, lane, h1);
        }
        gx0 = sum_lane_groups(gx0);
        gx1 = sum_lane_groups(gx1);
        if (g == 0 && active && grad_coordinates != nullptr) {
          grad_coordinates[2 * point] = gx0;
          grad_coordinates[2 * point + 1] = gx1;
        }
      }
      clock.mark(kClockLayer0);
      clock.count(kClockTiles);
    }
    // kRest: interior points past the last whole round of 64-point tiles, as 16-point tiles
    // whose rows are split over the 4 waves (split_tile), so a round that is not whole costs a
    // quarter tile on the slots that have one instead of a whole tile on some. The scratch
    // overlays the dW staging buffer: the barrier waits for the last 64-point tile's readers.
    // (A separate instantiation: with this loop in the kernel the compiler schedules the
    // 64-point loop differently, about 0.5 % slower, so whole rounds run without it.)
    if (kRest && tile < interior_end) {  // uniform per workgroup
      __syncthreads();
      const SplitScratch scratch{
          s_stage, reinterpret_cast<f4 (*)[kSplitWaves][4][kWave]>(s_stage + 3 * kTPlane),
          reinterpret_cast<float (*)[kTWave]>(s_stage + 3 * kTPlane + 2 * kSplitWaves * 4 * kWave * 4),
          reinterpret_cast<float (*)[2][kTile]>(s_stage + 3 * kTPlane +
                                                2 * kSplitWaves * 4 * kWave * 4 +
                                                kSplitWaves * kTWave)};
      int phase = 0;
      for (; tile < interior_end; tile += slots) {
        keep_lds_reads_in_loop();
        const int m_pick = opaque(m);
        const TileInputs in = next;
        if (tile + slots < tiles) {
          next = load_tile_inputs<kLoss, kRest>(coordinates, grad_output, grad_laplacian, batch, whole,
                                         seed, tile + slots, w, m);
        }
        const int64_t point = whole * kBwdTile + (tile - whole) * kTile + m;
        SplitSums sums{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        split_tile<kLoss>(s_w, s_small, scratch, phase, w, g, m_pick,
                          opaque(rows_off) + 1088 * w, opaque(cols_off) + 16 * w,
                          m_pick * kWRow + 4 * g, in.x0, in.x1, kLoss ? 0.f : in.a,
                          kLoss ? 0.f : in.b, kLoss ? in.a : 0.f, point < batch, false, point,
                          grad_coordinates, seed, acc.dw, acc.bh, sums);
        // Into this wave's owned-neuron lanes (owned_neuron): the wave's rows only; the point
        // sums shared by the 4 waves from wave 0 alone.
        const bool own = (m_pick >> 2) == w;
        acc.w0x += own ? sums.w0x : 0.f;
        acc.w0y += own ? sums.w0y : 0.f;
        acc.b0 += own ? sums.b0 : 0.f;
        acc.wout += own ? sums.wout : 0.f;
        if (w == 0) {
          acc.bout += sums.bout;
          acc.loss += sums.loss;
        }
        deliver(next);
      }
      clock.mark(kClockRest);
    }
    if (kLoss) {
      for (; tile < tiles; tile += slots) {  // boundary tiles (uniform per workgroup)
        keep_lds_reads_in_loop();
        const int m_pick = opaque(m);
        const TileInputs in = next;
        if (tile + slots < tiles) {
          next = load_tile_inputs<kLoss, kRest>(coordinates, grad_output, grad_laplacian, batch, whole, seed,
                                         tile + slots, w, m);
        }
        const int64_t point = (tile - seed.interior_tiles) * kTile + m;
        const bool active = point < seed.boundary_count;
        boundary_tile(s_w, s_small, s_stage, rows_off, cols_off, w, g, m_pick, in.x0, in.x1,
                      active, seed.boundary_scale, acc);
        deliver(next);
        clock.mark(kClockBoundary);
        clock.count(kClockBoundaryTiles);
      }
    }

    // ---- this slot's partial row: every entry written by exactly one lane ----
    // Non-temporal stores: the row is read once, by the reduction kernel, so it is streamed out
    // at once instead of waiting dirty in L2 for the write-back at the kernel's end (with every
    // workgroup's row dirty there, that write-back took about 3 us of a short call's tail).
    float* row = partials + static_cast<int64_t>(slot) * kRowStride;
    const int dw_lane = opaque((16 * w + 4 * g) * kHidden + m);
#pragma unroll
    for (int l = 0; l < 3; ++l) {
      float* wrow = row + kHiddenBase + l * kHiddenStride;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          __builtin_nontemporal_store(4.0f * acc.dw[l][nb][r], &wrow[dw_lane + r * kHidden + 16 * nb]);
        }
      }
      // dW: the sums are of d/d(4 W); bias sums are of zbar_v' = c^-1 zbar_v.
      if (g == 0) __builtin_nontemporal_store(kC * acc.bh[l], &wrow[kHidden * kHidden + 16 * w + m]);
    }
    // Per-wave sums (lane = owned neuron) combined over the 4 waves in a fixed order.
    __syncthreads();  // every wave is done with the staging buffer
    {
      float* comb = s_stage;  // [quantity][wave][neuron]
      const int o = owned_neuron(m, g);
      comb[(0 * kBwdWaves + w) * kHidden + o] = acc.w0x;
      comb[(1 * kBwdWaves + w) * kHidden + o] = acc.w0y;
      comb[(2 * kBwdWaves + w) * kHidden + o] = acc.b0;
      comb[(3 * kBwdWaves + w) * kHidden + o] = acc.wout;
      if (lane == 0) {
        s_red[0][w] = acc.bout;
        s_red[1][w] = acc.loss;
        s_red[2][w] = acc.bloss;
      }
      __syncthreads();
      const int q = threadIdx.x >> 6, n = threadIdx.x & 63;  // quantity (0..3), neuron
      const float* c4 = comb + q * kBwdWaves * kHidden + n;
      const float total = ((c4[0] + c4[kHidden]) + c4[2 * kHidden]) + c4[3 * kHidden];
      const int dst = q == 0 ? kInputs * n : q == 1 ? kInputs * n + 1 : q == 2 ? kLayer0Bias + n : kOutputBase + n;
      // dW0 / 2, db0 / c, dw_out
      __builtin_nontemporal_store((q == 2 ? kC : q == 3 ? 1.0f : 2.0f) * total, &row[dst]);
      if (threadIdx.x < (kLoss ? 3 : 1)) {
        const float* red = s_red[threadIdx.x];
        const int col = threadIdx.x == 0 ? kOutputBase + kHidden : kLossColumn + threadIdx.x - 1;
        __builtin_nontemporal_store(((red[0] + red[1]) + red[2]) + red[3], &row[col]);
      }
    }
    __syncthreads();  // s_red and the staging buffer are reused by the next slot
    clock.mark(kClockPartials);
  }
  clock.store(w);
}

// ---------------------------------------------------------------------------------------------
// Small-batch backward. backward_kernel carries 16 points per wave through the whole walk:
// 2,304 dependent MFMAs per 64-point workgroup tile, so a batch with at most one workgroup
// tile per CU costs that latency whatever its size. Here a workgroup of 4 waves runs one
// 16-point tile at a time and wave w owns rows 16 w .. 16 w + 15 of every layer: 64 MFMAs per
// layer for the forward re-run, 64 for dW and 64 for W^T zbar (576 per tile and wave).
//   * Layer outputs h and adjoints zbar go to the other waves lane to lane through LDS
//     (s_x, the register layout of forward_split_kernel), for the next product's B operand.
//   * dW contracts over the tile's points, which sit on the lane axis: h (all 64 rows, per
//     layer) and this wave's zbar are also stored transposed, [row][c][4 g + s] for point
//     4 s + g at pitch 68, so one 16-byte read gives a lane 4 points of one (row, c).
//   * Each wave owns distinct entries of the slot's partial row (its rows of every block), so
//     the partial row needs no combine across waves.
// Slots and the fixed-order reduction are those of backward_kernel with 16-point tiles. The
// choice between the two kernels depends only on the batch, so results do not depend on the
// device. The tanh-jet, adjoint and loss arithmetic is backward_kernel's; the sums over points
// are grouped differently, so the two kernels agree to rounding, not bitwise.
template <bool kLoss>
__global__ void __launch_bounds__(kSplitWaves * kWave, 1)
backward_split_kernel(const float* __restrict__ coordinates, const float* __restrict__ params,
                      const float* __restrict__ grad_output,
                      const float* __restrict__ grad_laplacian,
                      float* __restrict__ grad_coordinates, float* __restrict__ partials,
                      int64_t batch, int64_t tiles, int slots, LossSeed seed) {
  __shared__ __attribute__((aligned(16))) float s_w[3 * kPlane];
  __shared__ __attribute__((aligned(16))) float s_small[kSmallFloats];
  __shared__ __attribute__((aligned(16))) float s_ht[3 * kTPlane];  // h0, h1, h2 transposed
  __shared__ f4 s_x[2][kSplitWaves][4][kWave];                       // lane-major exchange
  __shared__ __attribute__((aligned(16))) float s_zt[kSplitWaves][kTWave];
  __shared__ float s_gx[kSplitWaves][2][kTile];
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  const int m = lane & 15;
  const int g = lane >> 4;
  // Per-point inputs of 16-point tiles (load_tile_inputs with no 64-point tiles): the first
  // slot's first tile's are read before the staging and each next tile's during the current
  // one, so no tile starts with a wait on global memory (a call here is a few tiles long).
  TileInputs next{0.f, 0.f, 0.f, 0.f};
  if (static_cast<int>(blockIdx.x) < slots) {
    next = load_tile_inputs<kLoss, true>(coordinates, grad_output, grad_laplacian, batch, 0, seed,
                                         blockIdx.x, w, m);
  }
  const float step_count = kLoss ? seed.step[0] : 0.0f;  // advanced below, as in backward_kernel
  stage_parameters<kSplitWaves * kWave>(params, s_w, s_small, threadIdx.x);
  __syncthreads();
  if (kLoss && blockIdx.x == 0 && threadIdx.x == 0) seed.step[0] = step_count + 1.0f;

  const int rows_off = lane_rows(m, g) + 1088 * w;  // W[16 w + m][.] (forward operand)
  const int cols_off = lane_cols(m, g) + 16 * w;    // W[.][16 w + m] (transposed operand)
  const int t_read = m * kWRow + 4 * g;             // transposed reads: row m, points 4 s + g

  const SplitScratch scratch{s_ht, s_x, s_zt, s_gx};
  int phase = 0;  // alternates the s_x buffers
  for (int slot = blockIdx.x; slot < slots; slot += gridDim.x) {
    f4 dw[3][4];
#pragma unroll
    for (int l = 0; l < 3; ++l) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) dw[l][nb] = zero4();
    }
    // Per-lane sums: bias[l] of row 16 w + m (all lane groups), the others of row
    // 16 w + 4 g + (m & 3).
    float bias[3] = {0.f, 0.f, 0.f};
    float g_w0x = 0.f, g_w0y = 0.f, g_b0 = 0.f, g_wout = 0.f, g_bout = 0.f;
    float g_loss = 0.f, g_bloss = 0.f;

    if (slot != static_cast<int>(blockIdx.x)) {
      next = load_tile_inputs<kLoss, true>(coordinates, grad_output, grad_laplacian, batch, 0,
                                           seed, slot, w, m);
    }
    for (int64_t tile = slot; tile < tiles; tile += slots) {
      keep_lds_reads_in_loop();
      const TileInputs in = next;
      if (tile + slots < tiles) {
        next = load_tile_inputs<kLoss, true>(coordinates, grad_output, grad_laplacian, batch, 0,
                                             seed, tile + slots, w, m);
      }
      const bool on_boundary = kLoss && tile >= seed.interior_tiles;  // uniform per workgroup
      const int64_t point = (on_boundary ? tile - seed.interior_tiles : tile) * kTile + m;
      const bool active = point < (on_boundary ? seed.boundary_count : batch);
      const float gu = kLoss ? 0.f : in.a, gl = kLoss ? 0.f : in.b, f = kLoss ? in.a : 0.f;

      SplitSums sums{g_w0x, g_w0y, g_b0, g_wout, g_bout, g_loss, g_bloss};
      split_tile<kLoss>(s_w, s_small, scratch, phase, w, g, m, rows_off, cols_off, t_read, in.x0,
                        in.x1, gu, gl, f, active, on_boundary, point, grad_coordinates, seed, dw,
                        bias, sums);
      g_w0x = sums.w0x;
      g_w0y = sums.w0y;
      g_b0 = sums.b0;
      g_wout = sums.wout;
      g_bout = sums.bout;
      g_loss = sums.loss;
      g_bloss = sums.bloss;
      deliver(next);
    }

    // ---- this slot's partial row: each wave writes its own rows ----
    float* row = partials + static_cast<int64_t>(slot) * kRowStride;
    const int dw_lane = opaque((16 * w + 4 * g) * kHidden + m);
#pragma unroll
    for (int l = 0; l < 3; ++l) {
      float* wrow = row + kHiddenBase + l * kHiddenStride;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) wrow[dw_lane + r * kHidden + 16 * nb] = 4.0f * dw[l][nb][r];
      }
      if (g == 0) wrow[kHidden * kHidden + 16 * w + m] = kC * bias[l];
    }
    if (m < 4) {
      const int n = 16 * w + 4 * g + m;
      row[kInputs * n] = 2.0f * g_w0x;
      row[kInputs * n + 1] = 2.0f * g_w0y;
      row[kLayer0Bias + n] = kC * g_b0;
      row[kOutputBase + n] = g_wout;
    }
    if (w == 0 && lane == 0) {
      row[kOutputBase + kHidden] = g_bout;
      if (kLoss) {
        row[kLossColumn] = g_loss;
        row[kLossColumn + 1] = g_bloss;
      }
    }
  }
}

constexpr int kPerGroup = kMaxSlots / kReduceGroups;  // slots per group of the fixed tree

// Column k's entries of group `group`'s slots, in slot order, as loaded: slot and column are
// clamped to a written row, and fixed_tree_total drops what lies beyond them. The 16 loads are
// issued unconditionally, where this is called, and waited for once, in fixed_tree_total:
// behind per-slot branches the compiler had waited for the first load, and for everything
// issued before it, before it issued the other 15.
__device__ __forceinline__ void load_group_column(const float* __restrict__ partials, int slots,
                                                  int k, int columns, int group,
                                                  float (&v)[kPerGroup]) {
  const int column = k < columns ? k : 0;
#pragma unroll
  for (int i = 0; i < kPerGroup; ++i) {
    const int slot = group * kPerGroup + i;
    v[i] = partials[static_cast<int64_t>(slot < slots ? slot : slots - 1) * kRowStride + column];
  }
}

// The fixed-tree total of column k from load_group_column's entries: each group's entries in
// slot order, then the 16 group sums in group order; complete in the threads of group 0. Slots
// at or beyond `slots` add +0.0f, and a column >= `columns` sums to +0.0f.
__device__ __forceinline__ float fixed_tree_total(float (&v)[kPerGroup], int slots, int k,
                                                  int columns, float (*s_part)[64], int group,
                                                  int col) {
  // An empty asm that reads and writes the 16 values: the loads cannot sink past it (into
  // per-slot branches around the selects below), so they stay where they were issued.
  __asm__ volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                   "+v"(v[6]), "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]),
                   "+v"(v[12]), "+v"(v[13]), "+v"(v[14]), "+v"(v[15]));
  static_assert(kPerGroup == 16, "the asm above names 16 values");
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < kPerGroup; ++i) {
    const int slot = group * kPerGroup + i;
    acc += k < columns && slot < slots ? v[i] : 0.0f;
  }
  s_part[group][col] = acc;
  __syncthreads();
  float total = 0.0f;
  if (group == 0) {
#pragma unroll
    for (int i = 0; i < kReduceGroups; ++i) total += s_part[i][col];
  }
  return total;
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
  float v[kPerGroup];
  load_group_column(partials, slots, k, kParameterCount, group, v);
  const float total = fixed_tree_total(v, slots, k, kParameterCount, s_part, group, col);
  if (group == 0 && k < kParameterCount) grad[k] = total;
}

// Adam (torch.optim.Adam, amsgrad = False, maximize = False) on the flat parameter buffer.
struct AdamArgs {
  float* params;
  float* exp_avg;
  float* exp_avg_sq;
  const float* step;  // already advanced for this step by the gradient kernel
  float* loss;        // mean r^2 + w mean u_b^2
  float* grad;        // optional copy of the summed gradient (nullptr: none)
  double lr, beta1, beta2, eps, weight_decay;
  float inv_batch;       // fl(1 / B)
  float inv_boundary;    // fl(1 / B_b), 0 without boundary points
  float boundary_weight; // fl(w)
};

// The fixed-tree gradient sum of reduce_partials_kernel, then the Adam update of each
// parameter in the same thread, so the summed gradient never goes through memory. Element
// arithmetic follows torch's multi-tensor Adam (torch/optim/adam.py, _multi_tensor_adam):
//   g += wd p;  m = lerp(m, g, 1 - b1);  v = v b2 + (1 - b2) g g;
//   p += -(lr / bc1) m / (sqrt(v) / sqrt(bc2) + eps),  bc_i = 1 - b_i^t,
// with the bias corrections in double and every tensor operation rounded to float. Columns
// kLossColumn and kLossColumn + 1 give loss = fl(sum r^2 / B) + fl(w fl(sum u_b^2 / B_b)).
__global__ void __launch_bounds__(kReduceGroups * 64)
reduce_adam_kernel(const float* __restrict__ partials, int slots, AdamArgs a) {
  __shared__ float s_part[kReduceGroups][64];
  __shared__ float s_loss[2];
  const int col = threadIdx.x & 63;
  const int group = threadIdx.x >> 6;
  const int k = blockIdx.x * 64 + col;
  // The Adam state is read before the partial rows, so the two memory round trips overlap.
  const bool updates = group == 0 && k < kParameterCount;
  float p = 0.0f, m = 0.0f, v = 0.0f;
  if (updates) {
    p = a.params[k];
    m = a.exp_avg[k];
    v = a.exp_avg_sq[k];
  }
  const float step_count = a.step[0];
  float parts[kPerGroup];
  load_group_column(partials, slots, k, kLossColumn + 2, group, parts);
  // The bias corrections (two double-precision powers, a long dependent chain) are formed in
  // the updating wave while the partial rows are in flight, not after their sum.
  float step_size = 0.0f, bc2_sqrt = 1.0f;
  if (updates) {
    const double t = static_cast<double>(step_count);
    const double bc1 = 1.0 - pow(a.beta1, t);
    const double bc2 = 1.0 - pow(a.beta2, t);
    step_size = static_cast<float>(-(a.lr / bc1));
    bc2_sqrt = static_cast<float>(sqrt(bc2));
  }
  const float total = fixed_tree_total(parts, slots, k, kLossColumn + 2, s_part, group, col);
  if (group == 0 && (k == kLossColumn || k == kLossColumn + 1)) s_loss[k - kLossColumn] = total;
  __syncthreads();
  if (group != 0) return;
  if (k == kLossColumn) {
    const float interior = s_loss[0] * a.inv_batch;
    a.loss[0] = a.inv_boundary != 0.0f ? interior + a.boundary_weight * (s_loss[1] * a.inv_boundary)
                                       : interior;
    return;
  }
  if (!updates) return;
  if (a.grad) a.grad[k] = total;
  const float w1 = static_cast<float>(1.0 - a.beta1);
  const float b2 = static_cast<float>(a.beta2);
  const float w2 = static_cast<float>(1.0 - a.beta2);
  const float eps = static_cast<float>(a.eps);
  const float wd = static_cast<float>(a.weight_decay);

  float g = total;
  if (wd != 0.0f) g = g + wd * p;
  m = m + w1 * (g - m);  // lerp with weight < 0.5
  v = v * b2;
  v = v + w2 * g * g;
  const float denom = sqrtf(v) / bc2_sqrt + eps;
  p = p + step_size * m / denom;
  a.exp_avg[k] = m;
  a.exp_avg_sq[k] = v;
  a.params[k] = p;
}

__global__ void fill_zero_kernel(float* __restrict__ out, int64_t n) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (k < n) out[k] = 0.0f;
}

// ---------------------------------------------------------------------------------------------
// Host side.

// Forward workgroup: 12 waves, 3 per SIMD (152 VGPRs each), about 1 % faster than 8 waves at 64K
// and 256K points; a CU's 16 tiles per 64K still split 4 per SIMD. The saving forward runs 8
// (launch_forward).
constexpr int kFwdWaves = 12;
constexpr int kSaveFwdWaves = 8;
constexpr int kSplitTilesPerCu = 2;  // forward_split_kernel up to this many tiles per CU

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

// Tiles of forward_kernel that run whole: all of them below one round of one tile per SIMD
// (4 per workgroup) or when the rounds are whole, otherwise the whole rounds; the rest run as
// split tiles. FUSED_HOAD_FWD_SPLIT_REST=0 (experiment knob, read per call) runs every tile
// whole.
int64_t forward_whole_tiles(int64_t tiles, int grid) {
  const int64_t round = 4 * static_cast<int64_t>(grid);
  if (const char* env = std::getenv("FUSED_HOAD_FWD_SPLIT_REST")) {
    if (std::atoi(env) == 0) return tiles;
  }
  if (tiles < round || tiles % round == 0) return tiles;
  return tiles - tiles % round;
}

// Compute units of the current device, queried once per device. The cache entries are atomic:
// calls from several host threads may fill the same entry (with the same value).
int current_device_cus(int* cus) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices] = {};
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(FHOAD_ERROR_DEVICE, "hipGetDevice: %s", hipGetErrorString(err));
  if (device >= 0 && device < kMaxDevices) {
    const int known = cached[device].load(std::memory_order_relaxed);
    if (known > 0) {
      *cus = known;
      return FHOAD_SUCCESS;
    }
  }
  int count = 0;
  err = hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device);
  if (err != hipSuccess) {
    return fail(FHOAD_ERROR_DEVICE, "hipDeviceGetAttribute: %s", hipGetErrorString(err));
  }
  if (count < 1) count = 1;
  if (device >= 0 && device < kMaxDevices) cached[device].store(count, std::memory_order_relaxed);
  *cus = count;
  return FHOAD_SUCCESS;
}

// Workspaces and saved-layer buffers must be 16-byte aligned (part of the ABI: hipMalloc and
// torch allocations are).
int check_workspace_alignment(const void* workspace, const char* what = "workspace") {
  if (reinterpret_cast<uintptr_t>(workspace) % alignof(f4) != 0) {
    return fail(FHOAD_ERROR_MISALIGNED, "%s must be 16-byte aligned", what);
  }
  return FHOAD_SUCCESS;
}

int64_t backward_tiles(int64_t batch) { return (batch + kBwdTile - 1) / kBwdTile; }

int slots_for_tiles(int64_t tiles) { return static_cast<int>(std::min<int64_t>(tiles, kMaxSlots)); }

int backward_slots(int64_t batch) { return slots_for_tiles(backward_tiles(batch)); }

// Workspace of the gradient kernels for `slots` slots: one partial row per slot.
constexpr size_t workspace_bytes_for(int slots) {
  return static_cast<size_t>(slots) * kRowStride * sizeof(float);
}

// Scratch of fhoad_forward_laplacian_backward_noalloc: a file-scope device array, one per GPU
// (each device that loads this code object holds its own copy until the process ends). It is
// sized for kMaxSlots slots, the most any batch uses (both gradient kernels cap their slots
// at kMaxSlots), so every batch fits. Host code never passes `scratch` itself to a kernel:
// the name is a host-side stand-in, and the device address comes from hipGetSymbolAddress
// (noalloc_scratch below).
constexpr size_t kNoAllocScratchBytes = workspace_bytes_for(kMaxSlots);
static_assert(kNoAllocScratchBytes % sizeof(float) == 0, "the scratch holds whole partial rows");
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

int64_t split_tiles(int64_t points) { return (points + kTile - 1) / kTile; }

// Interior tiles of backward_kernel for `batch` points over `slots` slots: 64-point tiles in
// whole rounds of `slots` (`whole` of them), then the remaining points as 16-point tiles whose
// rows are split over the waves (`total` counts both). Below one whole round, or when the
// rounds are whole, every tile is a 64-point one.
struct InteriorTiles {
  int64_t whole, total;
};

InteriorTiles interior_tiles_for(int64_t batch, int slots) {
  const int64_t t64 = backward_tiles(batch);
  const int64_t rounds = t64 / slots;
  if (rounds == 0 || t64 % slots == 0) return {t64, t64};
  const int64_t whole = rounds * slots;
  return {whole, whole + split_tiles(batch - whole * kBwdTile)};
}

// Gradient kernel for `batch` interior and `boundary_count` boundary points:
// backward_split_kernel up to kSplitBwdMaxTiles 16-point tiles, chosen from the batch alone
// so that results do not depend on the device. FUSED_HOAD_BWD_SPLIT=0 / 1 (experiment knob,
// read per call) forces either kernel.
bool use_split_backward(int64_t batch, int64_t boundary_count) {
  if (const char* env = std::getenv("FUSED_HOAD_BWD_SPLIT")) return std::atoi(env) != 0;
  return split_tiles(batch) + split_tiles(boundary_count) <= kSplitBwdMaxTiles;
}

// Workspace for either gradient kernel: one partial row per slot, for the larger slot count of
// the two (a knob can force either kernel).
size_t gradient_workspace_bytes(int64_t batch, int64_t boundary_count) {
  const int64_t boundary_tiles = split_tiles(boundary_count);
  return workspace_bytes_for(slots_for_tiles(
      std::max(backward_tiles(batch), split_tiles(batch)) + boundary_tiles));
}

// Persistent grid of the gradient kernel: one workgroup per CU, at most one per slot.
// FUSED_HOAD_BWD_BLOCKS caps it, as in the reference (fused_backward.cu:873-880). Here it
// changes only which workgroup computes a slot, never the arithmetic, so gradients stay
// bitwise identical.
int backward_grid(int slots, int* grid) {
  int cus = 0;
  if (int st = current_device_cus(&cus)) return st;
  *grid = std::min(slots, cus);
  if (const char* env = std::getenv("FUSED_HOAD_BWD_BLOCKS")) {
    const long cap = std::atol(env);
    if (cap > 0) *grid = static_cast<int>(std::min<long>(*grid, cap));
  }
  return FHOAD_SUCCESS;
}

// Device address of this device's `scratch`, looked up once per device (with that device
// current, on the first no-allocation call there) and kept per device: each GPU holds its own
// copy of the array at its own address. The cache entries are atomic, so calls from several
// host threads may fill one (with the same address).
int noalloc_scratch(void** out) {
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> addresses[kMaxDevices] = {};
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(FHOAD_ERROR_DEVICE, "hipGetDevice: %s", hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices) {
    return fail(FHOAD_ERROR_DEVICE, "device %d is beyond the %d devices the scratch table covers",
                device, kMaxDevices);
  }
  void* address = addresses[device].load(std::memory_order_acquire);
  if (address == nullptr) {
    // The first call on a device may come while the caller captures a HIP graph (the callers
    // this entry point is for): the lookup, which may load the code object on this device, runs
    // in the relaxed capture mode, so a global-mode capture in progress neither rejects it nor
    // is invalidated by it. The thread's mode is restored afterwards.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    err = hipThreadExchangeStreamCaptureMode(&mode);
    if (err != hipSuccess) {
      return fail(FHOAD_ERROR_DEVICE, "hipThreadExchangeStreamCaptureMode: %s", hipGetErrorString(err));
    }
    const hipError_t lookup = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    err = hipThreadExchangeStreamCaptureMode(&mode);
    if (lookup != hipSuccess || address == nullptr) {
      return fail(FHOAD_ERROR_DEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(lookup));
    }
    if (err != hipSuccess) {
      return fail(FHOAD_ERROR_DEVICE, "hipThreadExchangeStreamCaptureMode: %s", hipGetErrorString(err));
    }
    addresses[device].store(address, std::memory_order_release);
  }
  *out = address;
  return FHOAD_SUCCESS;
}

// Backward call on a workspace of `workspace_bytes` bytes (checked by the caller).
int launch_backward(const float* coordinates, const float* parameters, const float* grad_output,
                    const float* grad_laplacian, float* grad_parameters, float* grad_coordinates,
                    void* workspace, int64_t batch, hipStream_t hs, const void* saved = nullptr);

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

extern "C" int fhoad_check_device(void* stream) {
  hipError_t err = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(FHOAD_ERROR_DEVICE, "hipStreamSynchronize: %s", hipGetErrorString(err));
  unsigned status = 0;
  err = hipMemcpyFromSymbol(&status, HIP_SYMBOL(g_device_status), sizeof(status), 0, hipMemcpyDeviceToHost);
  if (err != hipSuccess) return fail(FHOAD_ERROR_DEVICE, "reading the device status: %s", hipGetErrorString(err));
  if (status == 0) return FHOAD_SUCCESS;
  const unsigned zero = 0;
  err = hipMemcpyToSymbol(HIP_SYMBOL(g_device_status), &zero, sizeof(zero), 0, hipMemcpyHostToDevice);
  if (err != hipSuccess) return fail(FHOAD_ERROR_DEVICE, "clearing the device status: %s", hipGetErrorString(err));
  return fail(FHOAD_ERROR_DEVICE,
              "a forward split tile's wave gave up waiting for its quad (status 0x%x): that tile's u "
              "and Laplacian were written as NaN",
              status);
}

#ifdef FHOAD_PHASE_CLOCK
// Measurement build only: the shape of backward_kernel's phase-clock table
// ([workgroups][waves][fields] of uint64), its reset and its copy to the host.
extern "C" void fhoad_phase_clock_shape(int* workgroups, int* waves, int* fields) {
  *workgroups = kClockWorkgroups;
  *waves = kBwdWaves;
  *fields = kClockFields;
}

extern "C" int fhoad_phase_clock_reset(void) {
  static const unsigned long long zeros[kClockWorkgroups * kBwdWaves * kClockFields] = {};
  hipError_t err = hipDeviceSynchronize();
  if (err == hipSuccess) err = hipMemcpyToSymbol(HIP_SYMBOL(g_phase_clock), zeros, sizeof(zeros));
  if (err != hipSuccess) return fail(FHOAD_ERROR_DEVICE, "resetting the phase clock: %s", hipGetErrorString(err));
  return FHOAD_SUCCESS;
}

extern "C" int fhoad_phase_clock_read(unsigned long long* out) {
  hipError_t err = hipDeviceSynchronize();
  if (err == hipSuccess) {
    err = hipMemcpyFromSymbol(out, HIP_SYMBOL(g_phase_clock), sizeof(g_phase_clock), 0,
                              hipMemcpyDeviceToHost);
  }
  if (err != hipSuccess) return fail(FHOAD_ERROR_DEVICE, "reading the phase clock: %s", hipGetErrorString(err));
  return FHOAD_SUCCESS;
}
#endif

namespace fhoad {
namespace {

// The forward launch shared by fhoad_forward_laplacian and fhoad_forward_laplacian_saving
// (kSave: the kernels also write the hidden-layer outputs to `saved`). batch > 0.
template <bool kSave>
int launch_forward(const float* coordinates, const float* parameters, float* output,
                   float* laplacian, void* saved, int64_t batch, hipStream_t hs) {
  int cus = 0;
  if (int st = current_device_cus(&cus)) return st;
  const int64_t tiles = (batch + kTile - 1) / kTile;
  const int grid = static_cast<int>(std::min<int64_t>(tiles, cus));
  f4* saved_f4 = static_cast<f4*>(saved);
  // Below kSplitTilesPerCu tiles per CU the split kernel runs each tile on a CU's 4 SIMDs.
  // FUSED_HOAD_FWD_SPLIT=0 / 1 (experiment knob, read per call) forces either kernel.
  const char* split_env = std::getenv("FUSED_HOAD_FWD_SPLIT");
  const bool split = split_env ? std::atoi(split_env) != 0 : tiles <= kSplitTilesPerCu * cus;
  if (split) {
    const int split_grid = static_cast<int>(std::min<int64_t>(tiles, kSplitTilesPerCu * cus));
    hipLaunchKernelGGL(forward_split_kernel<kSave>, dim3(split_grid), dim3(kSplitWaves * kWave), 0,
                       hs, coordinates, parameters, output, laplacian, batch, tiles, saved_f4);
    return check_launch("forward_split_kernel");
  }
  const int64_t whole = forward_whole_tiles(tiles, grid);
  // Waves per workgroup: 12 for the forward; 8 for the saving forward, whose 48 KB of stores per
  // tile slowed the 12-wave form more (64K points: 69 against 60 us; the plain forward 51.1
  // against 51.6 us). FUSED_HOAD_FWD_WAVES=8 / 12 (experiment knob, read per call) forces either.
  int waves = kSave ? kSaveFwdWaves : kFwdWaves;
  if (const char* env = std::getenv("FUSED_HOAD_FWD_WAVES")) {
    const int forced = std::atoi(env);
    if (forced == 8 || forced == 12) waves = forced;
  }
  // Polls per quad meeting before a split tile's wave gives up. FUSED_HOAD_QUAD_SPIN_LIMIT
  // (test knob, read per call) lowers it; 0 makes every meeting give up at once, so the tests can
  // check the timeout path (device status word, NaN outputs) with every kernel exiting normally.
  int spin_limit = kQuadSpinLimit;
  if (const char* env = std::getenv("FUSED_HOAD_QUAD_SPIN_LIMIT")) {
    spin_limit = static_cast<int>(std::min<long>(std::max<long>(std::atol(env), 0), kQuadSpinLimit));
  }
  if (waves == 8) {
    hipLaunchKernelGGL((forward_kernel<8, kSave>), dim3(grid), dim3(8 * kWave), 0, hs, coordinates,
                       parameters, output, laplacian, batch, whole, tiles, saved_f4, spin_limit);
  } else {
    hipLaunchKernelGGL((forward_kernel<kFwdWaves, kSave>), dim3(grid), dim3(kFwdWaves * kWave), 0,
                       hs, coordinates, parameters, output, laplacian, batch, whole, tiles,
                       saved_f4, spin_limit);
  }
  return check_launch("forward_kernel");
}

}  // namespace
}  // namespace fhoad

extern "C" int fhoad_forward_laplacian(const float* coordinates, const float* parameters,
                                       float* output, float* laplacian, int64_t batch,
                                       int version, void* stream) {
  if (version < 0 || version > 5) return fail(FHOAD_ERROR_INVALID_VERSION, "version must be 0 to 5");
  if (batch < 0) return fail(FHOAD_ERROR_INVALID_VALUE, "batch must be non-negative");
  if (batch == 0) return FHOAD_SUCCESS;
  if (!coordinates || !parameters || !output || !laplacian) {
    return fail(FHOAD_ERROR_INVALID_VALUE, "null device pointer");
  }
  return launch_forward<false>(coordinates, parameters, output, laplacian, nullptr, batch,
                               static_cast<hipStream_t>(stream));
}

extern "C" size_t fhoad_saved_layers_size(int64_t batch) {
  if (batch <= 0) return 0;
  // Unsigned, and saturated: a batch whose buffer would not fit in size_t gets SIZE_MAX, which
  // no buffer can hold, so the saving forward rejects it.
  constexpr uint64_t kTileBytes = static_cast<uint64_t>(kSavedF4PerTile) * sizeof(f4);
  const uint64_t tiles = (static_cast<uint64_t>(batch) + kTile - 1) / kTile;
  if (tiles > SIZE_MAX / kTileBytes) return SIZE_MAX;
  return static_cast<size_t>(tiles * kTileBytes);
}

extern "C" int fhoad_forward_laplacian_saving(const float* coordinates, const float* parameters,
                                              float* output, float* laplacian, void* saved,
                                              size_t saved_bytes, int64_t batch, int version,
                                              void* stream) {
  if (version < 0 || version > 5) return fail(FHOAD_ERROR_INVALID_VERSION, "version must be 0 to 5");
  if (batch < 0) return fail(FHOAD_ERROR_INVALID_VALUE, "batch must be non-negative");
  if (batch == 0) return FHOAD_SUCCESS;
  if (!coordinates || !parameters || !output || !laplacian) {
    return fail(FHOAD_ERROR_INVALID_VALUE, "null device pointer");
  }
  const size_t needed = fhoad_saved_layers_size(batch);
  if (!saved || saved_bytes < needed) {
    return fail(FHOAD_ERROR_WORKSPACE, "saved-layer buffer holds %zu bytes, %zu needed", saved_bytes,
                needed);
  }
  if (int st = check_workspace_alignment(saved, "saved-layer buffer")) return st;
  return launch_forward<true>(coordinates, parameters, output, laplacian, saved, batch,
                              static_cast<hipStream_t>(stream));
}

extern "C" size_t fhoad_backward_workspace_size(int64_t batch) {
  if (batch <= 0) return 0;
  return gradient_workspace_bytes(batch, 0);
}

extern "C" size_t fhoad_poisson_adam_step_workspace_size(int64_t batch, int64_t boundary_count) {
  if (batch <= 0 || boundary_count < 0) return 0;
  return gradient_workspace_bytes(batch, boundary_count);
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
  if (!coordinates) return fail(FHOAD_ERROR_INVALID_VALUE, "null device pointer");
  const size_t needed = fhoad_backward_workspace_size(batch);
  if (!workspace || workspace_bytes < needed) {
    return fail(FHOAD_ERROR_WORKSPACE, "workspace holds %zu bytes, %zu needed", workspace_bytes,
                needed);
  }
  if (int st = check_workspace_alignment(workspace)) return st;
  return launch_backward(coordinates, parameters, grad_output, grad_laplacian, grad_parameters,
                         grad_coordinates, workspace, batch, hs);
}

extern "C" int fhoad_forward_laplacian_backward_noalloc(
    const float* coordinates, const float* parameters, const float* grad_output,
    const float* grad_laplacian, float* grad_parameters, float* grad_coordinates, int64_t batch,
    int version, void* stream) {
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
  if (!coordinates) return fail(FHOAD_ERROR_INVALID_VALUE, "null device pointer");
  const size_t needed = fhoad_backward_workspace_size(batch);
  if (needed > kNoAllocScratchBytes) {
    return fail(FHOAD_ERROR_WORKSPACE, "batch %lld needs %zu bytes of scratch, the static scratch holds %zu",
                static_cast<long long>(batch), needed, kNoAllocScratchBytes);
  }
  void* device_scratch = nullptr;
  if (int st = noalloc_scratch(&device_scratch)) return st;
  return launch_backward(coordinates, parameters, grad_output, grad_laplacian, grad_parameters,
                         grad_coordinates, device_scratch, batch, hs);
}

extern "C" int fhoad_forward_laplacian_backward_saved(
    const float* coordinates, const float* parameters, const void* saved, size_t saved_bytes,
    const float* grad_output, const float* grad_laplacian, float* grad_parameters,
    float* grad_coordinates, void* workspace, size_t workspace_bytes, int64_t batch, int version,
    void* stream) {
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
  if (!coordinates) return fail(FHOAD_ERROR_INVALID_VALUE, "null device pointer");
  const size_t saved_needed = fhoad_saved_layers_size(batch);
  if (!saved || saved_bytes < saved_needed) {
    return fail(FHOAD_ERROR_WORKSPACE, "saved-layer buffer holds %zu bytes, %zu needed",
                saved_bytes, saved_needed);
  }
  if (int st = check_workspace_alignment(saved, "saved-layer buffer")) return st;
  const size_t needed = fhoad_backward_workspace_size(batch);
  if (!workspace || workspace_bytes < needed) {
    return fail(FHOAD_ERROR_WORKSPACE, "workspace holds %zu bytes, %zu needed", workspace_bytes,
                needed);
  }
  if (int st = check_workspace_alignment(workspace)) return st;
  return launch_backward(coordinates, parameters, grad_output, grad_laplacian, grad_parameters,
                         grad_coordinates, workspace, batch, hs, saved);
}

namespace fhoad {
namespace {

// saved: the saving forward's layer outputs for this batch (fhoad_saved_layers_size bytes), or
// null to re-run the forward. Batches the small-batch kernel takes re-run it either way.
int launch_backward(const float* coordinates, const float* parameters, const float* grad_output,
                    const float* grad_laplacian, float* grad_parameters, float* grad_coordinates,
                    void* workspace, int64_t batch, hipStream_t hs, const void* saved) {
  float* partials = static_cast<float*>(workspace);
  const f4* saved_f4 = static_cast<const f4*>(saved);
  const int64_t saved_tiles = (batch + kTile - 1) / kTile;
  int slots = 0, grid = 0;
  if (use_split_backward(batch, 0)) {
    const int64_t tiles = split_tiles(batch);
    slots = slots_for_tiles(tiles);
    if (int st = backward_grid(slots, &grid)) return st;
    hipLaunchKernelGGL(backward_split_kernel<false>, dim3(grid), dim3(kSplitWaves * kWave), 0, hs,
                       coordinates, parameters, grad_output, grad_laplacian, grad_coordinates,
                       partials, batch, tiles, slots, LossSeed{});
    if (int st = check_launch("backward_split_kernel")) return st;
  } else {
    slots = backward_slots(batch);
    if (int st = backward_grid(slots, &grid)) return st;
    const InteriorTiles it = interior_tiles_for(batch, slots);
    const dim3 block(kBwdWaves * kWave);
    if (it.whole != it.total && saved) {
      hipLaunchKernelGGL((backward_kernel<false, true, true>), dim3(grid), block, 0, hs,
                         coordinates, parameters, grad_output, grad_laplacian, grad_coordinates,
                         partials, batch, it.whole, it.total, slots, LossSeed{}, saved_f4,
                         saved_tiles);
    } else if (it.whole != it.total) {
      hipLaunchKernelGGL((backward_kernel<false, true, false>), dim3(grid), block, 0, hs,
                         coordinates, parameters, grad_output, grad_laplacian, grad_coordinates,
                         partials, batch, it.whole, it.total, slots, LossSeed{}, nullptr,
                         int64_t{0});
    } else if (saved) {
      hipLaunchKernelGGL((backward_kernel<false, false, true>), dim3(grid), block, 0, hs,
                         coordinates, parameters, grad_output, grad_laplacian, grad_coordinates,
                         partials, batch, it.whole, it.total, slots, LossSeed{}, saved_f4,
                         saved_tiles);
    } else {
      hipLaunchKernelGGL((backward_kernel<false, false, false>), dim3(grid), block, 0, hs,
                         coordinates, parameters, grad_output, grad_laplacian, grad_coordinates,
                         partials, batch, it.whole, it.total, slots, LossSeed{}, nullptr,
                         int64_t{0});
    }
    if (int st = check_launch("backward_kernel")) return st;
  }
  hipLaunchKernelGGL(reduce_partials_kernel, dim3((kParameterCount + 63) / 64),
                     dim3(kReduceGroups * 64), 0, hs, partials, slots, grad_parameters);
  return check_launch("reduce_partials_kernel");
}

}  // namespace
}  // namespace fhoad

extern "C" int fhoad_poisson_adam_step(const float* coordinates, const float* source,
                                       int64_t batch, const float* boundary,
                                       int64_t boundary_count, double boundary_weight,
                                       float* parameters, float* exp_avg, float* exp_avg_sq,
                                       float* step, float* loss, float* grad_parameters,
                                       float* grad_coordinates, void* workspace,
                                       size_t workspace_bytes, double lr, double beta1,
                                       double beta2, double eps, double weight_decay,
                                       void* stream) {
  if (batch <= 0) return fail(FHOAD_ERROR_INVALID_VALUE, "batch must be positive");
  if (boundary_count < 0) return fail(FHOAD_ERROR_INVALID_VALUE, "boundary_count must be non-negative");
  if (!coordinates || !source || !parameters || !exp_avg || !exp_avg_sq || !step || !loss ||
      (boundary_count > 0 && !boundary)) {
    return fail(FHOAD_ERROR_INVALID_VALUE, "null device pointer");
  }
  if (!(lr >= 0.0) || !(eps >= 0.0) || !(beta1 >= 0.0 && beta1 < 1.0) ||
      !(beta2 >= 0.0 && beta2 < 1.0) || !(weight_decay >= 0.0) || !(boundary_weight >= 0.0)) {
    return fail(FHOAD_ERROR_INVALID_VALUE,
                "Adam needs lr >= 0, eps >= 0, 0 <= betas < 1, weight_decay >= 0 and "
                "boundary_weight >= 0");
  }
  const size_t needed = fhoad_poisson_adam_step_workspace_size(batch, boundary_count);
  if (!workspace || workspace_bytes < needed) {
    return fail(FHOAD_ERROR_WORKSPACE, "workspace holds %zu bytes, %zu needed", workspace_bytes,
                needed);
  }
  if (int st = check_workspace_alignment(workspace)) return st;
  const bool split = use_split_backward(batch, boundary_count);
  const int slots = slots_for_tiles((split ? split_tiles(batch) : backward_tiles(batch)) +
                                    split_tiles(boundary_count));
  const InteriorTiles it =
      split ? InteriorTiles{0, split_tiles(batch)} : interior_tiles_for(batch, slots);
  const int64_t interior_tiles = it.total;
  const int64_t tiles = interior_tiles + split_tiles(boundary_count);  // 16-point boundary tiles
  int grid = 0;
  if (int st = backward_grid(slots, &grid)) return st;
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  const float inv_batch = 1.0f / static_cast<float>(batch);
  const float weight = static_cast<float>(boundary_weight);
  const float boundary_scale = boundary_count > 0 ? weight / static_cast<float>(boundary_count) : 0.0f;
  const float inv_boundary = boundary_count > 0 ? 1.0f / static_cast<float>(boundary_count) : 0.0f;
  float* partials = static_cast<float*>(workspace);
  const LossSeed seed{source, boundary, interior_tiles, boundary_count, inv_batch, boundary_scale, step};
  if (split) {
    hipLaunchKernelGGL(backward_split_kernel<true>, dim3(grid), dim3(kSplitWaves * kWave), 0, hs,
                       coordinates, parameters, nullptr, nullptr, grad_coordinates, partials,
                       batch, tiles, slots, seed);
    if (int st = check_launch("backward_split_kernel")) return st;
  } else {
    if (it.whole != it.total) {
      hipLaunchKernelGGL((backward_kernel<true, true, false>), dim3(grid), dim3(kBwdWaves * kWave),
                         0, hs, coordinates, parameters, nullptr, nullptr, grad_coordinates,
                         partials, batch, it.whole, tiles, slots, seed, nullptr, int64_t{0});
    } else {
      hipLaunchKernelGGL((backward_kernel<true, false, false>), dim3(grid), dim3(kBwdWaves * kWave),
                         0, hs, coordinates, parameters, nullptr, nullptr, grad_coordinates,
                         partials, batch, it.whole, tiles, slots, seed, nullptr, int64_t{0});
    }
    if (int st = check_launch("backward_kernel")) return st;
  }
  const AdamArgs args{parameters, exp_avg, exp_avg_sq, step, loss, grad_parameters,
                      lr, beta1, beta2, eps, weight_decay, inv_batch, inv_boundary, weight};
  hipLaunchKernelGGL(reduce_adam_kernel, dim3((kLossColumn + 2 + 63) / 64),
                     dim3(kReduceGroups * 64), 0, hs, partials, slots, args);
  return check_launch("reduce_adam_kernel");
}
