// Fused PPO minibatch gradient through the actor and critic MLPs.
//
// Reference: PPOAgent._update_batch, rl/deep/agents/ppo.py:141-169, with the
// networks of rl/deep/agents/common.py:16-28 (MLP: Linear-act-Linear-act-
// Linear; the reference uses ReLU, the benchmark's CartPole configuration tanh):
//     values = value(observations).squeeze(1)                     (:147)
//     logits = policy(observations)                                (:149)
//     ... the PPO loss of ppo.py:150-167 (row_math.hpp) ...
//     loss.backward()                                               (:169)
// One launch computes, for one minibatch (rows index[0..B) of the rollout
// arrays), the gradient of the loss with respect to every weight and bias of
// both networks; a second launch sums the per-workgroup partials in a fixed
// order (fp64) into the parameters' gradient tensors and forms the loss
// scalars.  clip_grad_norm_ + Adam (ppo.py:170-171) then run as
// ppo_adam_clip_f32 over those gradients.
//
// At the reference's sizes (4-64-64 or 4-128-128 networks, minibatches of
// 64-4096 rows) the torch sequence is ~35 small launches per minibatch;
// here it is two.  Layout: each block of kMlpRows = 16 minibatch rows is
// handled by two 256-thread workgroups, one per network (the actor's and
// the critic's forward, loss terms and backward share only the gathered
// observations).  Observations, activations and row gradients live in LDS;
// weights are read from global memory (a few KiB to 64 KiB per layer,
// L2-resident).  Every layer is a set of 16x16 output tiles on the matrix
// cores (v_mfma_f32_16x16x4f32, one tile per wave at a time): forward tiles
// over output units, input-gradient tiles over input units, weight-gradient
// tiles over (output, input) pairs summed over the 16 rows.  All arithmetic
// is fp32, as torch's; sums over the minibatch differ from torch's GEMM
// order only by rounding.
#include <float.h>
#include <stdlib.h>

#include "common.hpp"
#include "adam.hpp"
#include "grid_sync.hpp"
#include "cartpole_row.hpp"
#include "row_math.hpp"
#include "sample_row.hpp"

namespace ppo {
namespace {

constexpr int kMlpBlock = 256;
constexpr int kMlpRows = 16;
constexpr int kMlpMaxIn = 64;
constexpr int kMlpMaxA = 32;
constexpr int kMlpSums = 5;  // policy, value, entropy, approx-kl, clipfrac
constexpr int kMlpTensors = 12;  // weights and biases of the two 3-layer networks

struct MlpNet {
  const float* w[3];
  const float* b[3];
  float* gw[3];
  float* gb[3];
  int ldw[3];  // row stride of w[l] in floats (its input count in global memory)
};

// Offsets of one network's tensors inside a flat gradient partial.
struct NetOffsets {
  long w[3], b[3];
};

struct MlpArgs {
  MlpNet actor, critic;
  NetOffsets oa, oc;
  int D, A, act;
  const float* obs;
  long n;
  const int64_t* idx;  // may be null: rows 0..B-1
  long B;
  const void* actions;
  int act64;
  const float* old_lp;
  const float* adv;
  const float* ret;
  const float* old_val;
  // RowParams fields (row_math.hpp)
  float lo, hi, clip, vclip;
  int use_vclip;
  float vc, ec, inv_b;
  float* gpart;    // [nblocks][P]
  double* spart;   // [kMlpSums][nblocks]
  long P;
  long nblocks;
  float* scalars;
  // Reduction blocks are aligned to the 12 parameter tensors (tensor j =
  // 6 * net + 2 * layer + is_bias, actor first): tensor j owns reduction
  // blocks [tblk[j], tblk[j + 1]) and global parameters [toff[j],
  // toff[j] + tnum[j]).
  long tblk[kMlpTensors + 1];
  long toff[kMlpTensors];
  long tnum[kMlpTensors];
  double* sqpart;          // per reduction block: sum of squares of its gradients (or null)
  int64_t* step_counter;   // incremented once by reduction block 0 (or null)
};

template <int kAct>
__device__ __forceinline__ float act_fwd(float x) {
  if constexpr (kAct == PPO_ACT_TANH) return tanhf(x);
  else return x > 0.0f ? x : 0.0f;
}
// derivative from the activation's output y (torch tanh_backward /
// threshold_backward)
template <int kAct>
__device__ __forceinline__ float act_grad(float g, float y) {
  if constexpr (kAct == PPO_ACT_TANH) return g * (1.0f - y * y);
  else return y > 0.0f ? g : 0.0f;
}

// ---------------------------------------------------------------------------
// 16x16 MFMA tiles (v_mfma_f32_16x16x4f32, fp32 in and out).  Per step of 4
// along the contraction, lane l supplies A(l % 16, k0 + l / 16) and
// B(k0 + l / 16, l % 16); the result C(4 * (l / 16) + r, l % 16) is element r.
// Every GEMM here has one 16-row side (the workgroup's minibatch rows) and
// is cut into such tiles, spread over the workgroup's 4 waves.
// ---------------------------------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// LDS row stride of a [16][H] activation buffer: H + 2 floats, so a half-
// wave's operand reads (16 rows x 2 columns) fall in 32 distinct banks.
template <int H>
constexpr int act_ld() { return H + 2; }
constexpr int kXld = kMlpMaxIn + 2;   // observations [16][kXld]
constexpr int kZld = kMlpMaxA + 2;    // logits / dlogits [16][kZld]

// Forward tile: out[r][n] = f(b[n] + sum_{k<K} in[r][k] W[n][k]) for the 16
// columns n in [16 tj, 16 tj + 16) below N (f = the activation, or identity
// for kAct < 0).  KC = K at compile time (0: runtime K): the lane's weight
// values are then loaded in one batch.
template <int KC, int kAct>
__device__ __forceinline__ void fwd_tile(const float* in, int ldin, int K,
                                         const float* __restrict__ W, int ldw,
                                         const float* __restrict__ b, int N, float* out,
                                         int ldout, int tj) {
  const int l = threadIdx.x % kWave, i = l % 16, kk = l / 16;
  const int n = 16 * tj + i;
  const bool nok = n < N;
  const float* wrow = W + (long)(nok ? n : 0) * ldw;
  v4f c = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (KC > 0) {
    // contraction order permuted so that each lane's weights are contiguous:
    // in step (q, e) lane (i, kk) contributes k = 16 q + 4 kk + e, its weight
    // row read as one float4 per q
    static_assert(KC % 16 == 0, "compile-time K must be a multiple of 16");
    float4 bw[KC / 16];
#pragma unroll
    for (int q = 0; q < KC / 16; ++q)
      bw[q] = nok ? *reinterpret_cast<const float4*>(wrow + 16 * q + 4 * kk)
                  : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int q = 0; q < KC / 16; ++q) {
      const float* ir = in + i * ldin + 16 * q + 4 * kk;
      c = mfma4(ir[0], bw[q].x, c);
      c = mfma4(ir[1], bw[q].y, c);
      c = mfma4(ir[2], bw[q].z, c);
      c = mfma4(ir[3], bw[q].w, c);
    }
  } else {
    for (int k0 = 0; k0 < K; k0 += 4) {
      const int k = k0 + kk;
      const float av = k < K ? in[i * ldin + k] : 0.0f;
      const float bv = (k < K && nok) ? wrow[k] : 0.0f;
      c = mfma4(av, bv, c);
    }
  }
  if (nok) {
    const float bias = b[n];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float v = c[r] + bias;
      if constexpr (kAct >= 0) out[(4 * kk + r) * ldout + n] = act_fwd<kAct>(v);
      else out[(4 * kk + r) * ldout + n] = v;
    }
  }
}

// Input-gradient tile of a layer with H inputs: gin[r][k] = act'(h[r][k]) *
// sum_{m<M} d[r][m] W[m][k] for k in [16 tj, 16 tj + 16).  MC = M at compile
// time (0: runtime M).  W rows are read along k: coalesced.
template <int H, int MC, int kAct>
__device__ __forceinline__ void back_tile(const float* d, int ldd, int M,
                                          const float* __restrict__ W, int ldw, const float* h,
                                          float* gin, int tj) {
  constexpr int ld = act_ld<H>();
  const int l = threadIdx.x % kWave, i = l % 16, kk = l / 16;
  const int col = 16 * tj + i;
  v4f c = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (MC > 0) {
    float bw[MC / 4];
#pragma unroll
    for (int q = 0; q < MC / 4; ++q) bw[q] = W[(long)(4 * q + kk) * ldw + col];
#pragma unroll
    for (int q = 0; q < MC / 4; ++q) c = mfma4(d[i * ldd + 4 * q + kk], bw[q], c);
  } else {
    for (int m0 = 0; m0 < M; m0 += 4) {
      const int m = m0 + kk;
      const float av = m < M ? d[i * ldd + m] : 0.0f;
      const float bv = m < M ? W[(long)m * ldw + col] : 0.0f;
      c = mfma4(av, bv, c);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 4 * kk + r;
    gin[row * ld + col] = act_grad<kAct>(c[r], h[row * ld + col]);
  }
}

// Weight-gradient tile: gw[m][k] = sum over the 16 rows r of d[r][m] in[r][k]
// for m in [16 ti, 16 ti + 16) below M and k in [16 tj, 16 tj + 16) below K,
// written to the workgroup's partial (row-major [M][K]).
__device__ __forceinline__ void wgrad_tile(const float* d, int ldd, int M, const float* in,
                                           int ldin, int K, float* __restrict__ gw, int ti,
                                           int tj) {
  const int l = threadIdx.x % kWave, i = l % 16, kk = l / 16;
  const int m = 16 * ti + i, k = 16 * tj + i;
  v4f c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = 4 * q + kk;
    const float av = m < M ? d[r * ldd + m] : 0.0f;
    const float bv = k < K ? in[r * ldin + k] : 0.0f;
    c = mfma4(av, bv, c);
  }
  if (k < K) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int mo = 16 * ti + 4 * kk + r;
      if (mo < M) gw[(long)mo * K + k] = c[r];
    }
  }
}

// Bias gradient: gb[m] = sum over the 16 rows of d[r][m], threads t < M of a
// kBlock-thread workgroup.
template <int kBlock>
__device__ __forceinline__ void bgrad(const float* d, int ldd, int M, float* __restrict__ gb) {
  for (int m = threadIdx.x; m < M; m += kBlock) {
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < kMlpRows; ++r) s += d[r * ldd + m];
    gb[m] = s;
  }
}

// One network's backward from the gradient d3 [16][M3] at its output:
// phase 1 (dW3, db3, gradient into the second hidden layer), phase 2 (dW2,
// db2, gradient into the first), phase 3 (dW1, db1).  LDS-only barriers
// between the phases (the gradient partials go to global memory and are read
// by the next kernel); phase 3 leaves without one (the caller's next phase
// must not write g1 before a barrier).
template <int H, int kAct, int kBlock>
__device__ __forceinline__ void net_backward(const MlpNet& net, const NetOffsets& o, float* gp,
                                             const float* d3, int ld3, int M3, const float* x,
                                             int D, const float* h1, const float* h2, float* g1,
                                             float* g2) {
  constexpr int ld = act_ld<H>();
  constexpr int NT = H / 16;
  const int w = threadIdx.x / kWave;
  constexpr int kWaves = kBlock / kWave;
  const int MT3 = (M3 + 15) / 16;
  // phase 1
  for (int t = w; t < MT3 * NT + NT; t += kWaves) {
    if (t < MT3 * NT) wgrad_tile(d3, ld3, M3, h2, ld, H, gp + o.w[2], t / NT, t % NT);
    else back_tile<H, 0, kAct>(d3, ld3, M3, net.w[2], net.ldw[2], h2, g2, t - MT3 * NT);
  }
  bgrad<kBlock>(d3, ld3, M3, gp + o.b[2]);
  lds_barrier();
  // phase 2
  for (int t = w; t < NT * NT + NT; t += kWaves) {
    if (t < NT * NT) wgrad_tile(g2, ld, H, h1, ld, H, gp + o.w[1], t / NT, t % NT);
    else back_tile<H, H, kAct>(g2, ld, H, net.w[1], net.ldw[1], h1, g1, t - NT * NT);
  }
  bgrad<kBlock>(g2, ld, H, gp + o.b[1]);
  lds_barrier();
  // phase 3
  const int DT = (D + 15) / 16;
  for (int t = w; t < NT * DT; t += kWaves)
    wgrad_tile(g1, ld, H, x, kXld, D, gp + o.w[0], t / DT, t % DT);
  bgrad<kBlock>(g1, ld, H, gp + o.b[0]);
}

// Forward of both networks for the workgroup's 16 rows x (observations in
// s_x): hidden activations into a1/a2 (actor) and c1/c2 (critic), logits into
// z [16][kZld], values into v [16].  Tiles (network, column tile) over the
// waves of a kBlock-thread workgroup; LDS-only barriers between the layers
// and after the last.
template <int H, int kAct, int kBlock = kMlpBlock>
__device__ __forceinline__ void mlp_forward(const MlpNet& actor, const MlpNet& critic,
                                            const float* x, int D, int A, float* a1, float* a2,
                                            float* c1, float* c2, float* z, float* v) {
  constexpr int ld = act_ld<H>();
  constexpr int NT = H / 16;
  constexpr int kWaves = kBlock / kWave;
  const int w = threadIdx.x / kWave;
  for (int t = w; t < 2 * NT; t += kWaves) {
    const MlpNet& net = t < NT ? actor : critic;
    fwd_tile<0, kAct>(x, kXld, D, net.w[0], net.ldw[0], net.b[0], H, t < NT ? a1 : c1, ld,
                      t % NT);
  }
  lds_barrier();
  for (int t = w; t < 2 * NT; t += kWaves) {
    const MlpNet& net = t < NT ? actor : critic;
    fwd_tile<H, kAct>(t < NT ? a1 : c1, ld, H, net.w[1], net.ldw[1], net.b[1], H,
                      t < NT ? a2 : c2, ld,
                      t % NT);
  }
  lds_barrier();
  const int AT = (A + 15) / 16;
  for (int t = w; t < AT + 1; t += kWaves) {
    if (t < AT) fwd_tile<H, -1>(a2, ld, H, actor.w[2], actor.ldw[2], actor.b[2], A, z, kZld, t);
    else fwd_tile<H, -1>(c2, ld, H, critic.w[2], critic.ldw[2], critic.b[2], 1, v, 1, 0);
  }
  lds_barrier();
}

// LDS copy of one network's weights and biases, read by every tile of
// every layer instead of global memory (H <= 64: it then fits beside the
// activations).  Rows are padded: layer 0 to D + 1 floats (the scalar
// first-layer reads of a tile's 16 rows fall in distinct banks), layers 1-2
// to H + 4 (float4 rows stay 16-byte aligned and a tile's rows start in
// different banks).  The copy is complete after the caller's next barrier.
template <int H>
constexpr int net_lds_floats() {
  return H * (kMlpMaxIn + 1) + H + H * (H + 4) + H + kMlpMaxA * (H + 4) + kMlpMaxA;
}
constexpr int kMlpLdsMaxH = 64;  // largest hidden size whose weights are staged

template <int H>
__device__ __forceinline__ MlpNet stage_net(const MlpNet& g, int D, int O, float* lds) {
  constexpr int ld1 = H + 4;
  const int ld0 = D + 1;
  float* w0 = lds;
  float* b0 = w0 + H * (kMlpMaxIn + 1);
  float* w1 = b0 + H;
  float* b1 = w1 + H * ld1;
  float* w2 = b1 + H;
  float* b2 = w2 + kMlpMaxA * ld1;
  constexpr int kW1Iters = (H * H / 4 + kMlpBlock - 1) / kMlpBlock;
  float4 t1[kW1Iters];
#pragma unroll
  for (int q = 0; q < kW1Iters; ++q) {
    const int e4 = threadIdx.x + q * kMlpBlock;
    t1[q] = e4 < H * H / 4 ? reinterpret_cast<const float4*>(g.w[1])[e4]
                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  for (int e = threadIdx.x; e < H * D; e += kMlpBlock) {
    const int r = e / D, c = e - r * D;
    w0[r * ld0 + c] = g.w[0][e];
  }
  for (int e4 = threadIdx.x; e4 < O * H / 4; e4 += kMlpBlock) {
    const int r = (4 * e4) / H, c = 4 * e4 - r * H;
    *reinterpret_cast<float4*>(w2 + r * ld1 + c) = reinterpret_cast<const float4*>(g.w[2])[e4];
  }
  if (threadIdx.x < H) {
    b0[threadIdx.x] = g.b[0][threadIdx.x];
    b1[threadIdx.x] = g.b[1][threadIdx.x];
  }
  if (threadIdx.x < O) b2[threadIdx.x] = g.b[2][threadIdx.x];
#pragma unroll
  for (int q = 0; q < kW1Iters; ++q) {
    const int e4 = threadIdx.x + q * kMlpBlock;
    if (e4 < H * H / 4) {
      const int r = (4 * e4) / H, c = 4 * e4 - r * H;
      *reinterpret_cast<float4*>(w1 + r * ld1 + c) = t1[q];
    }
  }
  MlpNet n = g;
  n.w[0] = w0;
  n.w[1] = w1;
  n.w[2] = w2;
  n.b[0] = b0;
  n.b[1] = b1;
  n.b[2] = b2;
  n.ldw[0] = ld0;
  n.ldw[1] = n.ldw[2] = ld1;
  return n;
}

// Forward of one network for the workgroup's 16 rows (observations in x):
// hidden activations into h1/h2, the O outputs into out [16][ldout].  Column
// tiles over the waves; LDS-only barriers between the layers and after the
// last.  kBlock threads.
template <int H, int kAct, int kBlock>
__device__ __forceinline__ void net_forward(const MlpNet& net, const float* x, int D, int O,
                                            float* h1, float* h2, float* out, int ldout) {
  constexpr int ld = act_ld<H>();
  constexpr int NT = H / 16;
  constexpr int kWaves = kBlock / kWave;
  const int w = threadIdx.x / kWave;
  for (int t = w; t < NT; t += kWaves)
    fwd_tile<0, kAct>(x, kXld, D, net.w[0], net.ldw[0], net.b[0], H, h1, ld, t);
  lds_barrier();
  for (int t = w; t < NT; t += kWaves)
    fwd_tile<H, kAct>(h1, ld, H, net.w[1], net.ldw[1], net.b[1], H, h2, ld, t);
  lds_barrier();
  for (int t = w; t < (O + 15) / 16; t += kWaves)
    fwd_tile<H, -1>(h2, ld, H, net.w[2], net.ldw[2], net.b[2], O, out, ldout, t);
  lds_barrier();
}

// One minibatch block of 16 rows is handled by two workgroups, 2b (actor)
// and 2b + 1 (critic): the networks share nothing but the gathered
// observations, so each workgroup runs one network's forward, its part of
// the per-row loss and its backward.  They write disjoint parts of the
// block's partials (the actor's and the critic's parameter columns of
// gpart row b; the policy / entropy / kl / clip-fraction sums and the value
// sum of spart column b), so the reduction sees exactly the values one
// workgroup doing both networks would leave.
//
// Workgroups of grad_block<H>() threads: at H = 128 (weights read from
// global memory, not staged in LDS) 16 waves, so that each wave takes a
// quarter of the tiles it would among 4 (measured on MI355X, minibatches of
// 128 rows: 20.1 -> 16.0 us per launch).
template <int H>
constexpr int grad_block() {
  return H == 128 ? 1024 : kMlpBlock;
}

template <int H, int kAct>
__global__ void __launch_bounds__(grad_block<H>()) mlp_cat_grad_kernel(MlpArgs a) {
  constexpr int kBlock = grad_block<H>();
  constexpr int R = kMlpRows;
  constexpr int ld = act_ld<H>();
  __shared__ float s_x[R * kXld];
  __shared__ float s_h1[R * ld], s_h2[R * ld];
  __shared__ float s_g1[R * ld], s_g2[R * ld];
  __shared__ float s_z[R * kZld];
  __shared__ float s_v[R];
  __shared__ long s_row[R];

  const int tid = threadIdx.x;
  const bool critic = (blockIdx.x & 1u) != 0u;
  const long blk = (long)(blockIdx.x >> 1);
  const long row0 = blk * R;
  const int D = a.D, A = a.A;
  // this workgroup's network, its weights staged in LDS when they fit
  constexpr bool kStage = H <= kMlpLdsMaxH;
  __shared__ __attribute__((aligned(16))) float s_w[kStage ? net_lds_floats<H>() : 1];
  static_assert(!kStage || kBlock == kMlpBlock, "stage_net strides by kMlpBlock");
  MlpNet net = critic ? a.critic : a.actor;
  if constexpr (kStage) net = stage_net<H>(net, D, critic ? 1 : A, s_w);
  // the loss inputs of row `tid` (tid < R) are loaded now, ahead of the
  // forward pass that precedes their use
  RowIn rin = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
  long raw_act = 0;
  if (tid < R) {
    const long i = row0 + tid;
    const long src = i < a.B ? (a.idx ? (long)a.idx[i] : i) : -1;
    s_row[tid] = src;
    const long sc = src >= 0 ? src : 0;
    if (critic) {
      rin.ret = a.ret[sc];
      rin.vo = a.use_vclip ? a.old_val[sc] : 0.0f;
    } else {
      rin.old_lp = a.old_lp[sc];
      rin.adv = a.adv[sc];
      raw_act = a.act64 ? (long)reinterpret_cast<const int64_t*>(a.actions)[sc]
                        : (long)reinterpret_cast<const int32_t*>(a.actions)[sc];
    }
  }
  lds_barrier();
  // gather the observation rows (padding rows past B are zeros)
  for (int e = tid; e < R * D; e += kBlock) {
    const int r = e / D, c = e - (e / D) * D;
    const long src = s_row[r];
    s_x[r * kXld + c] = (src >= 0 && src < a.n) ? a.obs[src * D + c] : 0.0f;
  }
  lds_barrier();

  if (critic) net_forward<H, kAct, kBlock>(net, s_x, D, 1, s_h1, s_h2, s_v, 1);
  else net_forward<H, kAct, kBlock>(net, s_x, D, A, s_h1, s_h2, s_z, kZld);

  // loss rows: logits -> dlogits in place (actor), value -> dvalue in place
  // (critic; the value terms do not depend on the log-prob, which is given
  // its old value here)
  double acc[kMlpSums] = {0.0, 0.0, 0.0, 0.0, 0.0};
  if (tid < R) {
    const long src = s_row[tid];
    float* zr = s_z + tid * kZld;
    if (src >= 0) {
      if (critic) {
        RowIn in = rin;
        in.v = s_v[tid];
        const RowOut o = ppo_row_math(a, in, in.old_lp);
        s_v[tid] = o.dval;
        acc[1] = (double)o.vl;
      } else {
        const int ai = (raw_act >= 0 && raw_act < A) ? (int)raw_act : -1;
        float H_ent;
        const RowOut o = cat_row_grad<kMlpMaxA>(a, zr, A, ai, a.ec * a.inv_b, rin, H_ent);
        acc[0] = (double)o.pol;
        acc[2] = (double)H_ent;
        acc[3] = (double)o.kl;
        acc[4] = (double)o.clipped;
      }
    } else if (critic) {
      s_v[tid] = 0.0f;
    } else {
      for (int j = 0; j < A; ++j) zr[j] = 0.0f;
    }
  }
  block_sum<kMlpSums>(acc);  // its barriers also publish s_z / s_v
  if (tid == 0) {
    if (critic) {
      a.spart[1 * a.nblocks + blk] = acc[1];
    } else {
      a.spart[0 * a.nblocks + blk] = acc[0];
#pragma unroll
      for (int k = 2; k < kMlpSums; ++k) a.spart[(long)k * a.nblocks + blk] = acc[k];
    }
  }

  float* gp = a.gpart + blk * a.P;
  if (critic)
    net_backward<H, kAct, kBlock>(net, a.oc, gp, s_v, 1, 1, s_x, D, s_h1, s_h2, s_g1, s_g2);
  else
    net_backward<H, kAct, kBlock>(net, a.oa, gp, s_z, kZld, A, s_x, D, s_h1, s_h2, s_g1, s_g2);
}

// Action selection through both networks (ppo.py:65-79 for N observations):
// the forward of mlp_cat_grad_kernel, then per row the inverse-CDF draw of
// sample_row.hpp at the caller's uniform.  Writes actions (int32), their
// log-probabilities and the critic's values, and copies the observations to
// obs_out when given (a rollout buffer row).  With `logits` set instead of
// `u` (ppo_mlp_forward_cat_f32), writes the actor's logits and the critic's
// values and draws nothing.
struct ActArgs {
  MlpNet actor, critic;
  int D, A;
  const float* obs;
  long N;
  const float* u;
  float* obs_out;
  int32_t* act;
  float* logp;
  float* val;
  float* logits;
};

// Threads of the one-workgroup act launch (at most kMlpRows rows, where the
// chain of dependent loads and barriers is the kernel's time): a wave per
// 16-column tile of both networks' hidden layers (2 H / 16 tiles), so that no
// wave works through several tiles one after another; at least kMlpBlock.
template <int H>
constexpr int act_wide_block() {
  return 2 * (H / 16) * kWave > kMlpBlock ? 2 * (H / 16) * kWave : kMlpBlock;
}

// kBlock threads: kMlpBlock, or act_wide_block<H>() for one workgroup.
template <int H, int kAct, int kBlock = kMlpBlock>
__global__ void __launch_bounds__(kBlock) mlp_act_cat_kernel(ActArgs a) {
  constexpr int R = kMlpRows;
  constexpr int ld = act_ld<H>();
  __shared__ float s_x[R * kXld];
  __shared__ float s_a1[R * ld], s_a2[R * ld], s_c1[R * ld], s_c2[R * ld];
  __shared__ float s_z[R * kZld];
  __shared__ float s_v[R];
  const int tid = threadIdx.x;
  const long row0 = (long)blockIdx.x * R;
  const int D = a.D;
  for (int e = tid; e < R * D; e += kBlock) {
    const int r = e / D, c = e - (e / D) * D;
    const long row = row0 + r;
    float x = 0.0f;
    if (row < a.N) {
      x = a.obs[row * D + c];
      if (a.obs_out) a.obs_out[row * D + c] = x;
    }
    s_x[r * kXld + c] = x;
  }
  const float u = a.u && tid < R && row0 + tid < a.N ? a.u[row0 + tid] : 0.0f;
  lds_barrier();
  mlp_forward<H, kAct, kBlock>(a.actor, a.critic, s_x, D, a.A, s_a1, s_a2, s_c1, s_c2, s_z,
                               s_v);
  if (a.logits) {
    for (int e = tid; e < R * a.A; e += kBlock) {
      const int r = e / a.A, j = e - r * a.A;
      if (row0 + r < a.N) a.logits[(row0 + r) * a.A + j] = s_z[r * kZld + j];
    }
    if (tid < R && row0 + tid < a.N) a.val[row0 + tid] = s_v[tid];
    return;
  }
  if (tid < R && row0 + tid < a.N) {
    int act;
    float lp;
    sample_cat_row(s_z + tid * kZld, a.A, u, act, lp);
    a.act[row0 + tid] = act;
    a.logp[row0 + tid] = lp;
    a.val[row0 + tid] = s_v[tid];
  }
}

// A whole CartPole rollout in one launch (ppo_cartpole_rollout_f32): the T
// steps of act (both forwards + the inverse-CDF draw, as mlp_act_cat_kernel)
// and environment step (cartpole_advance, as the stand-alone step kernel)
// for the workgroup's 16 environments.  The environments of a workgroup
// depend on nothing outside it, so the steps need no launch boundary; the
// observations stay in LDS from one step to the next and the state in the
// registers of threads 0-15.  The results equal those of the two kernels
// launched per step on the same uniforms (the same functions run in the
// same order).
struct RolloutArgs {
  MlpNet actor, critic;
  long N;
  int T, max_steps;
  const float* u_act;    // row t: N action uniforms, at u_act + t * su_act
  const float* u_reset;  // row t: N x 4 reset uniforms, at u_reset + t * su_reset
  long su_act, su_reset;
  double* state;
  int32_t* steps;
  const float* obs_in;
  float* obs_out;
  float* obs_buf;  // [T][N][4]
  int32_t* act_buf;
  float *logp_buf, *val_buf, *rew_buf;
  uint8_t* done_buf;
  float* ep_return;
  double* done_sum;
  int32_t* done_count;
};

constexpr int kCartpoleObs = 4;
constexpr int kCartpoleActions = 2;

template <int H, int kAct>
__global__ void __launch_bounds__(kMlpBlock) mlp_cartpole_rollout_kernel(RolloutArgs a) {
  constexpr int R = kMlpRows;
  constexpr int D = kCartpoleObs;
  constexpr int ld = act_ld<H>();
  __shared__ float s_x[R * kXld];
  __shared__ float s_a1[R * ld], s_a2[R * ld], s_c1[R * ld], s_c2[R * ld];
  __shared__ float s_z[R * kZld];
  __shared__ float s_v[R];
  // both networks' weights staged in LDS once for all T steps, when they fit
  constexpr bool kStage = H <= kMlpLdsMaxH;
  __shared__ __attribute__((aligned(16))) float s_wa[kStage ? net_lds_floats<H>() : 1];
  __shared__ __attribute__((aligned(16))) float s_wc[kStage ? net_lds_floats<H>() : 1];
  MlpNet actor = a.actor, critic = a.critic;
  if constexpr (kStage) {
    actor = stage_net<H>(a.actor, D, kCartpoleActions, s_wa);
    critic = stage_net<H>(a.critic, D, 1, s_wc);
  }
  const int tid = threadIdx.x;
  const long row0 = (long)blockIdx.x * R;
  const long n = row0 + tid;
  const bool mine = tid < R && n < a.N;  // thread tid steps environment n
  double st[4] = {0.0, 0.0, 0.0, 0.0};
  int steps = 0;
  float ep_ret = 0.0f;
  double dsum = 0.0;  // the tally as the stand-alone step keeps it
  int dcount = 0;
  if (mine) {
#pragma unroll
    for (int k = 0; k < 4; ++k) st[k] = a.state[n * 4 + k];
    steps = a.steps[n];
    if (a.ep_return) {
      ep_ret = a.ep_return[n];
      dsum = a.done_sum[n];
      dcount = a.done_count[n];
    }
  }
  if (tid < R) {
#pragma unroll
    for (int k = 0; k < D; ++k) s_x[tid * kXld + k] = mine ? a.obs_in[n * D + k] : 0.0f;
  }
  lds_barrier();
  for (int t = 0; t < a.T; ++t) {
    float u = 0.0f;
    float ur[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (mine) {
      u = a.u_act[(long)t * a.su_act + n];
#pragma unroll
      for (int k = 0; k < 4; ++k) ur[k] = a.u_reset[(long)t * a.su_reset + n * 4 + k];
#pragma unroll
      for (int k = 0; k < D; ++k) a.obs_buf[((long)t * a.N + n) * D + k] = s_x[tid * kXld + k];
    }
    mlp_forward<H, kAct>(actor, critic, s_x, D, kCartpoleActions, s_a1, s_a2, s_c1, s_c2, s_z,
                         s_v);
    if (mine) {
      int act;
      float lp;
      sample_cat_row(s_z + tid * kZld, kCartpoleActions, u, act, lp);
      const long o = (long)t * a.N + n;
      a.act_buf[o] = act;
      a.logp_buf[o] = lp;
      a.val_buf[o] = s_v[tid];
      const CartpoleStep r = cartpole_advance(st, act, steps, a.max_steps, ur);
      a.rew_buf[o] = 1.0f;
      a.done_buf[o] = r.done ? 1 : 0;
      const float ret = ep_ret + 1.0f;
      if (r.done) {
        dsum += (double)ret;
        dcount += 1;
      }
      ep_ret = r.done ? 0.0f : ret;
#pragma unroll
      for (int k = 0; k < D; ++k) s_x[tid * kXld + k] = (float)st[k];
    }
    lds_barrier();
  }
  if (mine) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      a.state[n * 4 + k] = st[k];
      a.obs_out[n * D + k] = (float)st[k];
    }
    a.steps[n] = steps;
    if (a.ep_return) {
      a.ep_return[n] = ep_ret;
      a.done_sum[n] = dsum;
      a.done_count[n] = dcount;
    }
  }
}

// Sum the per-workgroup gradient partials into the parameters' gradient
// tensors: a workgroup owns up to 64 consecutive parameters of one tensor;
// wave w of its kWaves sums partials w, w + kWaves, ... (fp64, kLoads loads
// in flight per step) and the wave sums are added in wave order, so the
// order is fixed for a given geometry (deterministic).  The partial rows are
// read from HBM at a stride of the whole parameter count, so the kernel is
// latency-bound: for >= 128 partial rows, 16 waves x 16 loads put a
// 4096-row minibatch's 256 rows in flight at once (update of T=2048 x N=64 in
// minibatches of 4096: 4.69 -> 4.37 ms); fewer rows keep 4 waves x 8 loads.
// With sqpart the workgroup also leaves the fp64 sum of the squares of the
// fp32 gradients it wrote (clip_grad_norm_'s per-tensor sums, in pieces).
// Workgroup 0 also forms the loss scalars.
constexpr int kRedCols = 64;
constexpr long kRedWideRows = 128;  // partial rows from which the wide geometry is used

__device__ __forceinline__ float* tensor_grad(const MlpArgs& a, int j) {
  const MlpNet& net = j < 6 ? a.actor : a.critic;
  const int l = (j % 6) / 2;
  return (j & 1) ? net.gb[l] : net.gw[l];
}

template <int kWaves, int kRedLoads>
__global__ void __launch_bounds__(kWaves * kWave) mlp_grad_reduce_kernel(MlpArgs a) {
  constexpr int kRedBlock = kWaves * kWave;
  __shared__ double s_sum[kWaves][kRedCols];
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const long blk = blockIdx.x;
  int j = 0;
  while (j + 1 < kMlpTensors && blk >= a.tblk[j + 1]) ++j;
  const long local = (blk - a.tblk[j]) * kRedCols + lane;
  const bool valid = local < a.tnum[j];
  const long pc = a.toff[j] + (valid ? local : 0);
  double s = 0.0;
  for (long b0 = w; b0 < a.nblocks; b0 += kRedLoads * kWaves) {
    float v[kRedLoads];
#pragma unroll
    for (int q = 0; q < kRedLoads; ++q) {
      const long b = b0 + (long)q * kWaves;
      v[q] = a.gpart[(b < a.nblocks ? b : 0) * a.P + pc];
    }
#pragma unroll
    for (int q = 0; q < kRedLoads; ++q)
      if (b0 + (long)q * kWaves < a.nblocks) s += (double)v[q];
  }
  s_sum[w][lane] = s;
  __syncthreads();
  if (w == 0) {
    double t = s_sum[0][lane];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) t += s_sum[k][lane];
    const float g = (float)t;
    if (valid) tensor_grad(a, j)[local] = g;
    if (a.sqpart) {
      const double sq = wave_sum(valid ? (double)g * (double)g : 0.0);
      if (lane == 0) a.sqpart[blk] = sq;
    }
  }
  if (blk == 0) {
    if (threadIdx.x == 0 && a.step_counter) *a.step_counter += 1;
    double tot[kMlpSums];
    for (int k = 0; k < kMlpSums; ++k) tot[k] = 0.0;
    for (long b = threadIdx.x; b < a.nblocks; b += kRedBlock)
      for (int k = 0; k < kMlpSums; ++k) tot[k] += a.spart[(long)k * a.nblocks + b];
    block_sum<kMlpSums>(tot);
    if (threadIdx.x == 0) {
      const double nb = (double)a.B;
      const float pol = (float)(tot[0] / nb);
      const float vl = (float)(tot[1] / nb);
      const float ent = (float)(tot[2] / nb);
      a.scalars[PPO_SCALAR_POLICY] = pol;
      a.scalars[PPO_SCALAR_VALUE] = vl;
      a.scalars[PPO_SCALAR_ENTROPY] = ent;
      a.scalars[PPO_SCALAR_APPROX_KL] = (float)(tot[3] / nb);
      a.scalars[PPO_SCALAR_CLIPFRAC] = (float)(tot[4] / nb);
      a.scalars[PPO_SCALAR_LOSS] = (pol + a.vc * vl) - a.ec * ent;
    }
  }
}

// The reduction, clip_grad_norm_ and Adam in one launch (ppo_mlp_cat_step_f32
// when the reduction grid is resident on the device at once).  Each
// workgroup sums its parameters' gradient partials as
// mlp_grad_reduce_kernel does and publishes the sum of squares of the fp32
// gradients to a slot (grid_sync.hpp: value-tagged 64-bit words, cleared by
// the owner before a start barrier); then every workgroup reads all slots
// and forms the per-tensor norms, the total norm and the clip coefficient
// in the order adam_update_kernel uses (wave w takes tensors w, w + kWaves,
// ...; lane l sums a tensor's partials l, l + 64, ... in fp64, then the wave
// tree; adam_coef_from_norms), and updates its parameters from registers.
// The results are bit-identical to the reduction + adam_update_kernel
// launches, with one dependent launch fewer per minibatch.
struct MlpAdamArgs {
  float* p[kMlpTensors];
  float* m[kMlpTensors];
  float* v[kMlpTensors];
  AdamScalars s;
  float* norm_out;
  uint64_t* sync;  // start barrier (kSyncWords words)
  uint64_t* sq;    // per reduction workgroup: its sum-of-squares slot
  uint64_t* epoch; // the workspace header's call counter (launch_tag)
  unsigned nonce;
  WaitCtl wc;      // poll limit and the device's wait-status word
};

template <int kWaves, int kRedLoads>
__global__ void __launch_bounds__(kWaves * kWave) mlp_reduce_adam_kernel(MlpArgs a,
                                                                         MlpAdamArgs u) {
  __shared__ double s_sum[kWaves][kRedCols];
  __shared__ float s_norm[kMlpTensors];
  __shared__ float s_coef;
  const int lane = threadIdx.x % kWave;
  const int w = threadIdx.x / kWave;
  const long blk = blockIdx.x;
  int j = 0;
  while (j + 1 < kMlpTensors && blk >= a.tblk[j + 1]) ++j;
  const long local = (blk - a.tblk[j]) * kRedCols + lane;
  const bool valid = local < a.tnum[j];
  const long li = valid ? local : 0;
  const long pc = a.toff[j] + li;
  // wave 0: this workgroup's parameters and moments (they do not depend on
  // the norm), the step count (read before arriving: workgroup 0 advances it
  // only once every workgroup has arrived), its slot emptied, arrival
  float pr = 0.0f, mr = 0.0f, vr = 0.0f;
  int64_t step0 = 0;
  unsigned tag = 0;  // (wave 0)
  uint64_t epoch = 0;
  if (w == 0) {
    pr = u.p[j][li];
    mr = u.m[j][li];
    vr = u.v[j][li];
    if (a.step_counter) step0 = *a.step_counter;
    tag = launch_tag(u.epoch, u.nonce, epoch);
    sync_start(u.sync, u.sq + blk, 1, tag);
  }
  double s = 0.0;
  for (long b0 = w; b0 < a.nblocks; b0 += kRedLoads * kWaves) {
    float x[kRedLoads];
#pragma unroll
    for (int q = 0; q < kRedLoads; ++q) {
      const long b = b0 + (long)q * kWaves;
      x[q] = a.gpart[(b < a.nblocks ? b : 0) * a.P + pc];
    }
#pragma unroll
    for (int q = 0; q < kRedLoads; ++q)
      if (b0 + (long)q * kWaves < a.nblocks) s += (double)x[q];
  }
  s_sum[w][lane] = s;
  __syncthreads();
  float g = 0.0f;
  if (w == 0) {
    double t = s_sum[0][lane];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) t += s_sum[k][lane];
    g = (float)t;
    const double sq = wave_sum(valid ? (double)g * (double)g : 0.0);
    if (lane == 0) slot_put(u.sq + blk, sq);
  }
  if (blk == 0) {
    double tot[kMlpSums];
    for (int k = 0; k < kMlpSums; ++k) tot[k] = 0.0;
    for (long b = threadIdx.x; b < a.nblocks; b += kWaves * kWave)
      for (int k = 0; k < kMlpSums; ++k) tot[k] += a.spart[(long)k * a.nblocks + b];
    block_sum<kMlpSums>(tot);
    if (threadIdx.x == 0) {
      const double nb = (double)a.B;
      const float pol = (float)(tot[0] / nb);
      const float vl = (float)(tot[1] / nb);
      const float ent = (float)(tot[2] / nb);
      a.scalars[PPO_SCALAR_POLICY] = pol;
      a.scalars[PPO_SCALAR_VALUE] = vl;
      a.scalars[PPO_SCALAR_ENTROPY] = ent;
      a.scalars[PPO_SCALAR_APPROX_KL] = (float)(tot[3] / nb);
      a.scalars[PPO_SCALAR_CLIPFRAC] = (float)(tot[4] / nb);
      a.scalars[PPO_SCALAR_LOSS] = (pol + a.vc * vl) - a.ec * ent;
    }
  }
  // A wait that gives up (grid not co-resident) may leave slots unread or
  // read before their owner emptied them: this workgroup then writes none of
  // its parameters, moments or gradients (and workgroup 0 neither the step
  // counter; the norm output reads NaN), and raises the wait-status word.
  int fail = 0;
  if (threadIdx.x == 0) {
    if (!res_wait(u.sync, tag, gridDim.x, u.wc.spin)) fail = 1;
    if (blk == 0) epoch_advance(u.epoch, epoch);
  }
  // (after the barrier every workgroup has arrived and emptied its slot)
  if (__syncthreads_or(fail)) {
    if (threadIdx.x == 0) {
      wait_report(u.wc.status);
      if (blk == 0 && u.norm_out) *u.norm_out = __builtin_nanf("");
    }
    return;
  }
  for (int kk = w; kk < kMlpTensors; kk += kWaves) {
    double acc = 0.0;
    for (long c = a.tblk[kk] + lane; c < a.tblk[kk + 1]; c += kWave)
      acc += slot_get(u.sq + c, u.wc.spin, fail);
    const double sk = wave_sum(acc);
    if (lane == 0) s_norm[kk] = (float)sqrt(sk);
  }
  if (__syncthreads_or(fail)) {
    if (threadIdx.x == 0) {
      wait_report(u.wc.status);
      if (blk == 0 && u.norm_out) *u.norm_out = __builtin_nanf("");
    }
    return;
  }
  if (blk == 0 && threadIdx.x == 0 && a.step_counter) *a.step_counter = step0 + 1;
  if (threadIdx.x == 0) {
    float norm;
    s_coef = adam_coef_from_norms(u.s, s_norm, kMlpTensors, norm);
    if (blk == 0 && u.norm_out) *u.norm_out = norm;
  }
  __syncthreads();
  if (w == 0 && valid) {
    AdamScalars sc = u.s;
    if (a.step_counter) adam_step_scalars_at(sc, (double)(step0 + 1));
    float gi, mi, vi, pi;
    adam_elem(sc, s_coef, g, mr, vr, pr, gi, mi, vi, pi);
    tensor_grad(a, j)[local] = gi;  // (clipped when clipping, as clip_grad_norm_ leaves it)
    u.p[j][local] = pi;
    u.m[j][local] = mi;
    u.v[j][local] = vi;
  }
}

long mlp_params(int D, int H, int O) { return (long)H * D + H + (long)H * H + H + (long)O * H + O; }

NetOffsets net_offsets(long base, int D, int H, int O) {
  NetOffsets o;
  o.w[0] = base;
  o.b[0] = o.w[0] + (long)H * D;
  o.w[1] = o.b[0] + H;
  o.b[1] = o.w[1] + (long)H * H;
  o.w[2] = o.b[1] + H;
  o.b[2] = o.w[2] + (long)O * H;
  return o;
}

struct MlpLayout {
  long P, nblocks, rblocks;
  int threads;  // of the gradient kernel's workgroups
  long tblk[kMlpTensors + 1], toff[kMlpTensors], tnum[kMlpTensors];
  size_t gpart, spart, sqpart, sync, total;
};

MlpLayout mlp_layout(long B, int D, int H, int A) {
  MlpLayout l;
  l.P = mlp_params(D, H, A) + mlp_params(D, H, 1);
  l.threads = H == 128 ? grad_block<128>() : kMlpBlock;
  l.nblocks = (B + kMlpRows - 1) / kMlpRows;
  const NetOffsets o[2] = {net_offsets(0, D, H, A), net_offsets(mlp_params(D, H, A), D, H, 1)};
  const int outs[2] = {A, 1};
  l.tblk[0] = 0;
  for (int j = 0; j < kMlpTensors; ++j) {
    const int net = j / 6, layer = (j % 6) / 2;
    const long in = layer == 0 ? D : H, out = layer == 2 ? outs[net] : H;
    l.toff[j] = (j & 1) ? o[net].b[layer] : o[net].w[layer];
    l.tnum[j] = (j & 1) ? out : out * in;
    l.tblk[j + 1] = l.tblk[j] + (l.tnum[j] + kRedCols - 1) / kRedCols;
  }
  l.rblocks = l.tblk[kMlpTensors];
  l.gpart = kHeaderBytes;
  l.spart = l.gpart + align_up((size_t)l.nblocks * l.P * sizeof(float), 256);
  l.sqpart = l.spart + align_up((size_t)kMlpSums * l.nblocks * sizeof(double), 256);
  l.sync = l.sqpart + align_up((size_t)l.rblocks * sizeof(double), 256);
  l.total = l.sync + kSyncWords * sizeof(uint64_t);
  return l;
}

template <int kAct>
const void* mlp_kernel_act(int H) {
  switch (H) {
    case 16: return (const void*)mlp_cat_grad_kernel<16, kAct>;
    case 32: return (const void*)mlp_cat_grad_kernel<32, kAct>;
    case 64: return (const void*)mlp_cat_grad_kernel<64, kAct>;
    case 128: return (const void*)mlp_cat_grad_kernel<128, kAct>;
    default: return nullptr;
  }
}

int act_wide_threads(int H) {
  switch (H) {
    case 64: return act_wide_block<64>();
    case 128: return act_wide_block<128>();
    default: return kMlpBlock;
  }
}

template <int kAct>
const void* act_kernel_act(int H, bool wide) {
  switch (H) {
    case 16: return (const void*)mlp_act_cat_kernel<16, kAct>;
    case 32: return (const void*)mlp_act_cat_kernel<32, kAct>;
    case 64:
      return wide ? (const void*)mlp_act_cat_kernel<64, kAct, act_wide_block<64>()>
                  : (const void*)mlp_act_cat_kernel<64, kAct>;
    case 128:
      return wide ? (const void*)mlp_act_cat_kernel<128, kAct, act_wide_block<128>()>
                  : (const void*)mlp_act_cat_kernel<128, kAct>;
    default: return nullptr;
  }
}

template <int kAct>
const void* rollout_kernel_act(int H) {
  switch (H) {
    case 16: return (const void*)mlp_cartpole_rollout_kernel<16, kAct>;
    case 32: return (const void*)mlp_cartpole_rollout_kernel<32, kAct>;
    case 64: return (const void*)mlp_cartpole_rollout_kernel<64, kAct>;
    case 128: return (const void*)mlp_cartpole_rollout_kernel<128, kAct>;
    default: return nullptr;
  }
}

bool mlp_net_weights_ok(const ppo_mlp3_f32* n) {
  if (!n) return false;
  for (int l = 0; l < 3; ++l)
    if (!n->weight[l] || !n->bias[l] || !aligned(n->weight[l], 16)) return false;
  return true;
}

bool mlp_net_ok(const ppo_mlp3_f32* n) {
  if (!n) return false;
  for (int l = 0; l < 3; ++l)
    if (!n->weight[l] || !n->bias[l] || !n->weight_grad[l] || !n->bias_grad[l]) return false;
  return true;
}

MlpNet to_net(const ppo_mlp3_f32* n, int D, int H) {
  MlpNet m;
  for (int l = 0; l < 3; ++l) {
    m.w[l] = n->weight[l];
    m.b[l] = n->bias[l];
    m.gw[l] = n->weight_grad[l];
    m.gb[l] = n->bias_grad[l];
  }
  m.ldw[0] = D;
  m.ldw[1] = m.ldw[2] = H;
  return m;
}

}  // namespace
}  // namespace ppo

extern "C" size_t ppo_mlp_cat_grad_workspace_bytes(int64_t B, int32_t obs_dim, int32_t hidden,
                                                    int32_t A) {
  using namespace ppo;
  if (B <= 0 || obs_dim <= 0 || hidden <= 0 || A <= 0) return kHeaderBytes;
  return mlp_layout(B, obs_dim, hidden, A).total;
}

namespace ppo {
namespace {

// Validation and argument setup shared by ppo_mlp_cat_grad_f32 and
// ppo_mlp_cat_step_f32; on PPO_OK, `kern`, `a` and `l` are ready to launch
// (B == 0 returns PPO_OK with kern null: nothing to do).
int mlp_setup(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic, int32_t obs_dim,
              int32_t hidden, int32_t A, int32_t activation, const float* observations,
              int64_t n, const int64_t* index, int64_t B, const void* actions,
              int actions_are_int64, const float* old_log_probs, const float* advantages,
              const float* returns, const float* old_values, const ppo_loss_params* params,
              float* scalars_out, void* workspace, size_t workspace_bytes, const void*& kern,
              MlpArgs& a, MlpLayout& l) {
  kern = nullptr;
  if (B < 0 || n < 0) return PPO_ERR_INVALID_ARG;
  if (obs_dim <= 0 || obs_dim > kMlpMaxIn || A <= 0 || A > kMlpMaxA) return PPO_ERR_UNSUPPORTED;
  if (activation != PPO_ACT_RELU && activation != PPO_ACT_TANH) return PPO_ERR_INVALID_ARG;
  const void* k = activation == PPO_ACT_TANH ? mlp_kernel_act<PPO_ACT_TANH>(hidden)
                                             : mlp_kernel_act<PPO_ACT_RELU>(hidden);
  if (!k) return PPO_ERR_UNSUPPORTED;
  if (!mlp_net_ok(actor) || !mlp_net_ok(critic) || !params || !scalars_out)
    return PPO_ERR_INVALID_ARG;
  if (B == 0) return PPO_OK;
  if (!observations || !actions || !old_log_probs || !advantages || !returns)
    return PPO_ERR_INVALID_ARG;
  if (B > (1L << 31) || n > (1L << 40)) return PPO_ERR_TOO_LARGE;
  if (!workspace || workspace_bytes < ppo_mlp_cat_grad_workspace_bytes(B, obs_dim, hidden, A))
    return PPO_ERR_WORKSPACE;
  for (int li = 0; li < 3; ++li)
    if (!aligned(actor->weight[li], 16) || !aligned(critic->weight[li], 16))
      return PPO_ERR_INVALID_ARG;
  l = mlp_layout(B, obs_dim, hidden, A);
  char* ws = static_cast<char*>(workspace);
  a = MlpArgs{};
  a.actor = to_net(actor, obs_dim, hidden);
  a.critic = to_net(critic, obs_dim, hidden);
  a.oa = net_offsets(0, obs_dim, hidden, A);
  a.oc = net_offsets(mlp_params(obs_dim, hidden, A), obs_dim, hidden, 1);
  a.D = obs_dim;
  a.A = A;
  a.act = activation;
  a.obs = observations;
  a.n = n;
  a.idx = index;
  a.B = B;
  a.actions = actions;
  a.act64 = actions_are_int64;
  a.old_lp = old_log_probs;
  a.adv = advantages;
  a.ret = returns;
  a.old_val = old_values;
  const RowParams rp = make_row_params(params, B);
  a.lo = rp.lo;
  a.hi = rp.hi;
  a.clip = rp.clip;
  a.vclip = rp.vclip;
  a.use_vclip = rp.use_vclip;
  if (a.use_vclip && !old_values) return PPO_ERR_INVALID_ARG;
  a.vc = rp.vc;
  a.ec = rp.ec;
  a.inv_b = rp.inv_b;
  a.gpart = reinterpret_cast<float*>(ws + l.gpart);
  a.spart = reinterpret_cast<double*>(ws + l.spart);
  a.P = l.P;
  a.nblocks = l.nblocks;
  a.scalars = scalars_out;
  for (int j = 0; j <= kMlpTensors; ++j) a.tblk[j] = l.tblk[j];
  for (int j = 0; j < kMlpTensors; ++j) {
    a.toff[j] = l.toff[j];
    a.tnum[j] = l.tnum[j];
  }
  a.sqpart = nullptr;
  a.step_counter = nullptr;
  kern = k;
  return PPO_OK;
}

// The gradient kernel (two workgroups per 16-row block) and the reduction.
int mlp_launch(const void* kern, MlpArgs& a, const MlpLayout& l, hipStream_t stream) {
  void* args[] = {&a};
  int st = hip_status(hipLaunchKernel(kern, dim3((unsigned)(2 * l.nblocks)), dim3(l.threads),
                                      args, 0, stream));
  if (st) return st;
  const bool wide = l.nblocks >= kRedWideRows;
  return hip_status(hipLaunchKernel(wide ? (const void*)mlp_grad_reduce_kernel<16, 16>
                                         : (const void*)mlp_grad_reduce_kernel<4, 8>,
                                    dim3((unsigned)l.rblocks), dim3(wide ? 1024 : 256), args, 0,
                                    stream));
}

}  // namespace
}  // namespace ppo

extern "C" int ppo_mlp_cat_grad_f32(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic,
                                    int32_t obs_dim, int32_t hidden, int32_t A,
                                    int32_t activation, const float* observations, int64_t n,
                                    const int64_t* index, int64_t B, const void* actions,
                                    int actions_are_int64, const float* old_log_probs,
                                    const float* advantages, const float* returns,
                                    const float* old_values, const ppo_loss_params* params,
                                    float* scalars_out, void* workspace, size_t workspace_bytes,
                                    void* stream_ptr) {
  using namespace ppo;
  const void* kern;
  MlpArgs a;
  MlpLayout l;
  const int st = mlp_setup(actor, critic, obs_dim, hidden, A, activation, observations, n, index,
                           B, actions, actions_are_int64, old_log_probs, advantages, returns,
                           old_values, params, scalars_out, workspace, workspace_bytes, kern, a,
                           l);
  if (st || !kern) return st;
  return mlp_launch(kern, a, l, reinterpret_cast<hipStream_t>(stream_ptr));
}

extern "C" int ppo_mlp_cat_step_f32(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic,
                                    int32_t obs_dim, int32_t hidden, int32_t A,
                                    int32_t activation, const float* observations, int64_t n,
                                    const int64_t* index, int64_t B, const void* actions,
                                    int actions_are_int64, const float* old_log_probs,
                                    const float* advantages, const float* returns,
                                    const float* old_values, const ppo_loss_params* params,
                                    float* const* exp_avg, float* const* exp_avg_sq,
                                    const ppo_adam_params* adam, float* scalars_out,
                                    float* grad_norm_out, void* workspace, size_t workspace_bytes,
                                    void* stream_ptr) {
  using namespace ppo;
  if (!exp_avg || !exp_avg_sq || !adam) return PPO_ERR_INVALID_ARG;
  for (int j = 0; j < kMlpTensors; ++j)
    if (!exp_avg[j] || !exp_avg_sq[j]) return PPO_ERR_INVALID_ARG;
  if ((!adam->step_counter && adam->step < 1) || !(adam->lr >= 0.0) || !(adam->eps >= 0.0))
    return PPO_ERR_INVALID_ARG;
  const void* kern;
  MlpArgs a;
  MlpLayout l;
  int st = mlp_setup(actor, critic, obs_dim, hidden, A, activation, observations, n, index, B,
                     actions, actions_are_int64, old_log_probs, advantages, returns, old_values,
                     params, scalars_out, workspace, workspace_bytes, kern, a, l);
  if (st || !kern) return st;
  a.sqpart = reinterpret_cast<double*>(static_cast<char*>(workspace) + l.sqpart);
  a.step_counter = adam->step_counter;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  // one launch for the reduction and the update when its grid is resident
  // (PPO_AMD_MLP_FUSED_ADAM=0 in the environment keeps two launches)
  const bool wide = l.nblocks >= kRedWideRows;
  const void* fused = wide ? (const void*)mlp_reduce_adam_kernel<16, 16>
                           : (const void*)mlp_reduce_adam_kernel<4, 8>;
  const int fused_threads = wide ? 1024 : 256;
  const char* env = getenv("PPO_AMD_MLP_FUSED_ADAM");
  if (!(env && env[0] == '0') && l.rblocks <= 0x7fffffffL &&
      resident_blocks(fused, fused_threads, 0, 0) >= l.rblocks) {
    MlpAdamArgs u = {};
    for (int j = 0; j < kMlpTensors; ++j) {
      const ppo_mlp3_f32* net = j < 6 ? actor : critic;
      const int li = (j % 6) / 2;
      u.p[j] = const_cast<float*>((j & 1) ? net->bias[li] : net->weight[li]);  // in place
      u.m[j] = exp_avg[j];
      u.v[j] = exp_avg_sq[j];
    }
    u.s = make_adam_scalars(adam);
    u.norm_out = grad_norm_out;
    u.sync = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + l.sync);
    u.sq = reinterpret_cast<uint64_t*>(a.sqpart);
    u.epoch = &reinterpret_cast<WsHeader*>(workspace)->epoch;
    u.nonce = next_nonce();
    if ((st = wait_ctl(u.wc))) return st;
    void* gargs[] = {&a};
    if ((st = hip_status(hipLaunchKernel(kern, dim3((unsigned)(2 * l.nblocks)), dim3(l.threads),
                                         gargs, 0, stream))))
      return st;
    void* fargs[] = {&a, &u};
    return hip_status(hipLaunchKernel(fused, dim3((unsigned)l.rblocks), dim3(fused_threads),
                                      fargs, 0, stream));
  }
  if ((st = mlp_launch(kern, a, l, stream))) return st;
  float* pp[kMlpTensors];
  float* gp[kMlpTensors];
  int64_t numel[kMlpTensors];
  for (int j = 0; j < kMlpTensors; ++j) {
    const ppo_mlp3_f32* net = j < 6 ? actor : critic;
    const int li = (j % 6) / 2;
    pp[j] = const_cast<float*>((j & 1) ? net->bias[li] : net->weight[li]);  // updated in place
    gp[j] = (j & 1) ? net->bias_grad[li] : net->weight_grad[li];
    numel[j] = l.tnum[j];
  }
  return launch_adam_presummed(kMlpTensors, pp, gp, exp_avg, exp_avg_sq, numel, adam, a.sqpart,
                               l.tblk, grad_norm_out, stream);
}

namespace ppo {
namespace {

// The device's address of `p`: itself for device memory, the mapped address
// for pinned host memory (hipHostMalloc / torch pin_memory), so that a kernel
// reads and writes it over the bus.
void* device_view(const void* p) {
  if (!p) return nullptr;
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();
    return const_cast<void*>(p);
  }
  if (attr.type != hipMemoryTypeHost) return const_cast<void*>(p);
  void* d = nullptr;
  if (hipHostGetDevicePointer(&d, const_cast<void*>(p), 0) != hipSuccess || !d) {
    (void)hipGetLastError();
    return const_cast<void*>(p);
  }
  return d;
}

int launch_act(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic, int32_t obs_dim,
               int32_t hidden, int32_t A, int32_t activation, ActArgs& a, void* stream_ptr) {
  if (a.N < 0) return PPO_ERR_INVALID_ARG;
  if (obs_dim <= 0 || obs_dim > kMlpMaxIn || A <= 0 || A > kMlpMaxA) return PPO_ERR_UNSUPPORTED;
  if (activation != PPO_ACT_RELU && activation != PPO_ACT_TANH) return PPO_ERR_INVALID_ARG;
  // (one workgroup: the wide form, measured on MI355X at H = 128: 9.6 -> 8.4 us)
  const bool wide = a.N <= kMlpRows;
  const void* kern = activation == PPO_ACT_TANH ? act_kernel_act<PPO_ACT_TANH>(hidden, wide)
                                                : act_kernel_act<PPO_ACT_RELU>(hidden, wide);
  if (!kern) return PPO_ERR_UNSUPPORTED;
  if (!mlp_net_weights_ok(actor) || !mlp_net_weights_ok(critic)) return PPO_ERR_INVALID_ARG;
  if (a.N == 0) return PPO_OK;
  if (!a.obs || !a.val) return PPO_ERR_INVALID_ARG;
  if (a.N > (1L << 31)) return PPO_ERR_TOO_LARGE;
  a.actor = to_net(actor, obs_dim, hidden);
  a.critic = to_net(critic, obs_dim, hidden);
  a.D = obs_dim;
  a.A = A;
  void* args[] = {&a};
  const long blocks = (a.N + kMlpRows - 1) / kMlpRows;
  const int threads = wide ? act_wide_threads(hidden) : kMlpBlock;
  return hip_status(hipLaunchKernel(kern, dim3((unsigned)blocks), dim3(threads), args, 0,
                                    reinterpret_cast<hipStream_t>(stream_ptr)));
}

}  // namespace
}  // namespace ppo

extern "C" int ppo_mlp_act_cat_f32(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic,
                                   int32_t obs_dim, int32_t hidden, int32_t A,
                                   int32_t activation, const float* observations, int64_t N,
                                   const float* uniforms, float* observations_out,
                                   int32_t* actions_out, float* log_probs_out,
                                   float* values_out, void* stream_ptr) {
  using namespace ppo;
  if (N > 0 && (!uniforms || !actions_out || !log_probs_out)) return PPO_ERR_INVALID_ARG;
  ActArgs a = {};
  a.obs = observations;
  a.N = N;
  a.u = uniforms;
  a.obs_out = observations_out;
  a.act = actions_out;
  a.logp = log_probs_out;
  a.val = values_out;
  return launch_act(actor, critic, obs_dim, hidden, A, activation, a, stream_ptr);
}

extern "C" int ppo_mlp_forward_cat_f32(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic,
                                       int32_t obs_dim, int32_t hidden, int32_t A,
                                       int32_t activation, const float* observations,
                                       int64_t N, float* logits_out, float* values_out,
                                       void* stream_ptr) {
  using namespace ppo;
  if (N > 0 && !logits_out) return PPO_ERR_INVALID_ARG;
  ActArgs a = {};
  a.obs = static_cast<const float*>(device_view(observations));
  a.N = N;
  a.logits = static_cast<float*>(device_view(logits_out));
  a.val = static_cast<float*>(device_view(values_out));
  return launch_act(actor, critic, obs_dim, hidden, A, activation, a, stream_ptr);
}

extern "C" int ppo_cartpole_rollout_f32(
    const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic, int32_t hidden, int32_t activation,
    int64_t N, int32_t T, int32_t max_steps, double* state, int32_t* steps,
    const float* observations, float* observations_out, const float* action_uniforms,
    int64_t action_uniforms_stride, const float* reset_uniforms, int64_t reset_uniforms_stride,
    float* obs_buf, int32_t* actions_buf, float* log_probs_buf, float* values_buf,
    float* rewards_buf, uint8_t* dones_buf, float* episode_return, double* completed_sum,
    int32_t* completed_count, void* stream_ptr) {
  using namespace ppo;
  if (N < 0 || T < 0 || max_steps < 1) return PPO_ERR_INVALID_ARG;
  if (activation != PPO_ACT_RELU && activation != PPO_ACT_TANH) return PPO_ERR_INVALID_ARG;
  const void* kern = activation == PPO_ACT_TANH ? rollout_kernel_act<PPO_ACT_TANH>(hidden)
                                                : rollout_kernel_act<PPO_ACT_RELU>(hidden);
  if (!kern) return PPO_ERR_UNSUPPORTED;
  if (!mlp_net_weights_ok(actor) || !mlp_net_weights_ok(critic)) return PPO_ERR_INVALID_ARG;
  if ((episode_return == nullptr) != (completed_sum == nullptr) ||
      (episode_return == nullptr) != (completed_count == nullptr))
    return PPO_ERR_INVALID_ARG;
  if (N == 0 || T == 0) return PPO_OK;
  if (!state || !steps || !observations || !observations_out || !action_uniforms ||
      !reset_uniforms || !obs_buf || !actions_buf || !log_probs_buf || !values_buf ||
      !rewards_buf || !dones_buf)
    return PPO_ERR_INVALID_ARG;
  if (action_uniforms_stride < N || reset_uniforms_stride < 4 * N) return PPO_ERR_INVALID_ARG;
  if (N > (1L << 31) || (long)T * N > (1L << 40)) return PPO_ERR_TOO_LARGE;
  RolloutArgs a = {};
  a.actor = to_net(actor, kCartpoleObs, hidden);
  a.critic = to_net(critic, kCartpoleObs, hidden);
  a.N = N;
  a.T = T;
  a.max_steps = max_steps;
  a.u_act = action_uniforms;
  a.u_reset = reset_uniforms;
  a.su_act = action_uniforms_stride;
  a.su_reset = reset_uniforms_stride;
  a.state = state;
  a.steps = steps;
  a.obs_in = observations;
  a.obs_out = observations_out;
  a.obs_buf = obs_buf;
  a.act_buf = actions_buf;
  a.logp_buf = log_probs_buf;
  a.val_buf = values_buf;
  a.rew_buf = rewards_buf;
  a.done_buf = dones_buf;
  a.ep_return = episode_return;
  a.done_sum = completed_sum;
  a.done_count = completed_count;
  void* args[] = {&a};
  const long blocks = (N + kMlpRows - 1) / kMlpRows;
  return hip_status(hipLaunchKernel(kern, dim3((unsigned)blocks), dim3(kMlpBlock), args, 0,
                                    reinterpret_cast<hipStream_t>(stream_ptr)));
}
