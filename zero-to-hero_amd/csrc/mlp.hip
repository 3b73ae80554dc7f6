// Fused PPO minibatch gradient through the actor and critic MLPs.
//
// Reference: PPOAgent._update_batch, rl/deep/agents/ppo.py:141-169, with the
// networks of rl/deep/agents/common.py:16-28 (MLP: Linear-act-Linear-act-
// Linear; the reference uses ReLU, BASELINE's CartPole config tanh):
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
// here it is two.  Layout: a 256-thread workgroup owns kMlpRows = 16 rows.
// Observations, activations and row gradients live in LDS; weights are read
// from global memory (a few KiB to 64 KiB per layer, L2-resident).  Hidden
// layers map thread t to output unit t % H and rows t / H + (256/H) i, so a
// wave's LDS reads of the layer input are broadcasts and its weight-row reads
// are per-lane rows; the backward maps threads to input units, so the
// weight-column reads are coalesced.  All arithmetic is fp32, as torch's;
// sums over the minibatch differ from torch's GEMM order only by rounding.
#include <float.h>

#include "common.hpp"
#include "row_math.hpp"

namespace ppo {
namespace {

constexpr int kMlpBlock = 256;
constexpr int kMlpRows = 16;
constexpr int kMlpMaxIn = 64;
constexpr int kMlpMaxA = 32;
constexpr int kMlpSums = 5;  // policy, value, entropy, approx-kl, clipfrac

struct MlpNet {
  const float* w[3];
  const float* b[3];
  float* gw[3];
  float* gb[3];
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

// Hidden layer forward: out[r][m] = act(b[m] + sum_k W[m][k] in[r][k]),
// M = H outputs, K inputs (K % 4 == 0 when kVecK).
template <int H, int kAct, bool kVecK>
__device__ __forceinline__ void fwd_hidden(const float* __restrict__ W, const float* __restrict__ b,
                                           const float* in, int K, float* out) {
  constexpr int G = kMlpBlock / H;
  constexpr int RPT = kMlpRows / G;
  const int m = threadIdx.x % H;
  const int g = threadIdx.x / H;
  float acc[RPT];
  const float bm = b[m];
#pragma unroll
  for (int i = 0; i < RPT; ++i) acc[i] = bm;
  const float* wr = W + (long)m * K;
  if constexpr (kVecK) {
    for (int k = 0; k < K; k += 4) {
      const float4 w = *reinterpret_cast<const float4*>(wr + k);
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const float4 x = *reinterpret_cast<const float4*>(in + (g + G * i) * K + k);
        acc[i] = fmaf(w.x, x.x, acc[i]);
        acc[i] = fmaf(w.y, x.y, acc[i]);
        acc[i] = fmaf(w.z, x.z, acc[i]);
        acc[i] = fmaf(w.w, x.w, acc[i]);
      }
    }
  } else {
    for (int k = 0; k < K; ++k) {
      const float w = wr[k];
#pragma unroll
      for (int i = 0; i < RPT; ++i) acc[i] = fmaf(w, in[(g + G * i) * K + k], acc[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) out[(g + G * i) * H + m] = act_fwd<kAct>(acc[i]);
}

// Output layer forward: out[r][m] = b[m] + sum_k W[m][k] h[r][k], M <= 32.
template <int H>
__device__ __forceinline__ void fwd_out(const float* __restrict__ W, const float* __restrict__ b,
                                        const float* h, int M, float* out) {
  for (int o = threadIdx.x; o < kMlpRows * M; o += kMlpBlock) {
    const int r = o / M, m = o - (o / M) * M;
    const float* wr = W + (long)m * H;
    float acc = b[m];
#pragma unroll 4
    for (int k = 0; k < H; k += 4) {
      const float4 w = *reinterpret_cast<const float4*>(wr + k);
      const float4 x = *reinterpret_cast<const float4*>(h + r * H + k);
      acc = fmaf(w.x, x.x, acc);
      acc = fmaf(w.y, x.y, acc);
      acc = fmaf(w.z, x.z, acc);
      acc = fmaf(w.w, x.w, acc);
    }
    out[r * M + m] = acc;
  }
}

// Weight and bias gradient partials of one layer: gW[m][k] = sum_r d[r][m]
// in[r][k], gb[m] = sum_r d[r][m] over the workgroup's rows.
__device__ __forceinline__ void grad_wb(const float* d, int M, const float* in, int K,
                                        float* __restrict__ gw, float* __restrict__ gb) {
  for (int o = threadIdx.x; o < M * K; o += kMlpBlock) {
    const int m = o / K, k = o - (o / K) * K;
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < kMlpRows; ++r) s = fmaf(d[r * M + m], in[r * K + k], s);
    gw[o] = s;
  }
  for (int m = threadIdx.x; m < M; m += kMlpBlock) {
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < kMlpRows; ++r) s += d[r * M + m];
    gb[m] = s;
  }
}

// Gradient into a hidden layer's output: din[r][k] = act'(h[r][k]) *
// sum_m d[r][m] W[m][k], K = H units, M outputs of the next layer.
template <int H, int kAct>
__device__ __forceinline__ void back_hidden(const float* d, int M, const float* __restrict__ W,
                                            const float* h, float* din) {
  constexpr int G = kMlpBlock / H;
  constexpr int RPT = kMlpRows / G;
  const int k = threadIdx.x % H;
  const int g = threadIdx.x / H;
  float acc[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) acc[i] = 0.0f;
  for (int m = 0; m < M; ++m) {
    const float w = W[(long)m * H + k];
#pragma unroll
    for (int i = 0; i < RPT; ++i) acc[i] = fmaf(d[(g + G * i) * M + m], w, acc[i]);
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = g + G * i;
    din[r * H + k] = act_grad<kAct>(acc[i], h[r * H + k]);
  }
}

template <int H, int kAct, typename ActT>
__global__ void __launch_bounds__(kMlpBlock) mlp_cat_grad_kernel(MlpArgs a) {
  constexpr int R = kMlpRows;
  // (16-byte aligned: the layers read them as float4)
  __shared__ __align__(16) float s_x[R * kMlpMaxIn];
  __shared__ __align__(16) float s_a1[R * H], s_a2[R * H], s_c1[R * H], s_c2[R * H];
  __shared__ __align__(16) float s_g1[R * H], s_g2[R * H];
  __shared__ __align__(16) float s_z[R * kMlpMaxA];
  __shared__ __align__(16) float s_v[R];
  __shared__ long s_row[R];

  const int tid = threadIdx.x;
  const long row0 = (long)blockIdx.x * R;
  const int D = a.D, A = a.A;
  if (tid < R) {
    const long i = row0 + tid;
    s_row[tid] = i < a.B ? (a.idx ? (long)a.idx[i] : i) : -1;
  }
  __syncthreads();
  // gather the observation rows (padding rows past B are zeros)
  for (int e = tid; e < R * D; e += kMlpBlock) {
    const int r = e / D, c = e - (e / D) * D;
    const long src = s_row[r];
    s_x[e] = (src >= 0 && src < a.n) ? a.obs[src * D + c] : 0.0f;
  }
  __syncthreads();

  // forward: both networks
  if (D % 4 == 0) {
    fwd_hidden<H, kAct, true>(a.actor.w[0], a.actor.b[0], s_x, D, s_a1);
    fwd_hidden<H, kAct, true>(a.critic.w[0], a.critic.b[0], s_x, D, s_c1);
  } else {
    fwd_hidden<H, kAct, false>(a.actor.w[0], a.actor.b[0], s_x, D, s_a1);
    fwd_hidden<H, kAct, false>(a.critic.w[0], a.critic.b[0], s_x, D, s_c1);
  }
  __syncthreads();
  fwd_hidden<H, kAct, true>(a.actor.w[1], a.actor.b[1], s_a1, H, s_a2);
  fwd_hidden<H, kAct, true>(a.critic.w[1], a.critic.b[1], s_c1, H, s_c2);
  __syncthreads();
  fwd_out<H>(a.actor.w[2], a.actor.b[2], s_a2, A, s_z);
  fwd_out<H>(a.critic.w[2], a.critic.b[2], s_c2, 1, s_v);
  __syncthreads();

  // loss rows: logits -> dlogits in place, value -> dvalue in place
  double acc[kMlpSums] = {0.0, 0.0, 0.0, 0.0, 0.0};
  if (tid < R) {
    const long src = s_row[tid];
    float* zr = s_z + tid * A;
    if (src >= 0) {
      RowIn in;
      in.old_lp = a.old_lp[src];
      in.adv = a.adv[src];
      in.ret = a.ret[src];
      in.v = s_v[tid];
      in.vo = a.use_vclip ? a.old_val[src] : 0.0f;
      const long raw = a.act64 ? (long)reinterpret_cast<const int64_t*>(a.actions)[src]
                               : (long)reinterpret_cast<const int32_t*>(a.actions)[src];
      const int ai = (raw >= 0 && raw < A) ? (int)raw : -1;
      float H_ent;
      const RowOut o = cat_row_grad<kMlpMaxA>(a, zr, A, ai, a.ec * a.inv_b, in, H_ent);
      s_v[tid] = o.dval;
      acc[0] = (double)o.pol;
      acc[1] = (double)o.vl;
      acc[2] = (double)H_ent;
      acc[3] = (double)o.kl;
      acc[4] = (double)o.clipped;
    } else {
      for (int j = 0; j < A; ++j) zr[j] = 0.0f;
      s_v[tid] = 0.0f;
    }
  }
  block_sum<kMlpSums>(acc);  // its barriers also publish s_z / s_v
  if (tid == 0) {
#pragma unroll
    for (int k = 0; k < kMlpSums; ++k) a.spart[(long)k * a.nblocks + blockIdx.x] = acc[k];
  }

  float* gp = a.gpart + (long)blockIdx.x * a.P;
  // actor backward
  grad_wb(s_z, A, s_a2, H, gp + a.oa.w[2], gp + a.oa.b[2]);
  back_hidden<H, kAct>(s_z, A, a.actor.w[2], s_a2, s_g2);
  __syncthreads();
  grad_wb(s_g2, H, s_a1, H, gp + a.oa.w[1], gp + a.oa.b[1]);
  back_hidden<H, kAct>(s_g2, H, a.actor.w[1], s_a1, s_g1);
  __syncthreads();
  grad_wb(s_g1, H, s_x, D, gp + a.oa.w[0], gp + a.oa.b[0]);
  __syncthreads();
  // critic backward
  grad_wb(s_v, 1, s_c2, H, gp + a.oc.w[2], gp + a.oc.b[2]);
  back_hidden<H, kAct>(s_v, 1, a.critic.w[2], s_c2, s_g2);
  __syncthreads();
  grad_wb(s_g2, H, s_c1, H, gp + a.oc.w[1], gp + a.oc.b[1]);
  back_hidden<H, kAct>(s_g2, H, a.critic.w[1], s_c1, s_g1);
  __syncthreads();
  grad_wb(s_g1, H, s_x, D, gp + a.oc.w[0], gp + a.oc.b[0]);
}

// Sum the per-workgroup gradient partials (fixed order, fp64) into the
// parameters' gradient tensors; workgroup 0 also forms the loss scalars.
__global__ void __launch_bounds__(kMlpBlock) mlp_grad_reduce_kernel(MlpArgs a) {
  const long p = (long)blockIdx.x * kMlpBlock + threadIdx.x;
  if (p < a.P) {
    double s = 0.0;
    for (long b = 0; b < a.nblocks; ++b) s += (double)a.gpart[b * a.P + p];
    // which tensor p falls in: offsets ascend actor w0 b0 w1 b1 w2 b2, critic ...
    const MlpNet* nets[2] = {&a.actor, &a.critic};
    const NetOffsets* offs[2] = {&a.oa, &a.oc};
    float* dst = nullptr;
#pragma unroll
    for (int n = 0; n < 2; ++n)
#pragma unroll
      for (int l = 0; l < 3; ++l) {
        if (p >= offs[n]->w[l] && p < offs[n]->b[l]) dst = nets[n]->gw[l] + (p - offs[n]->w[l]);
        const long bend = (l < 2) ? offs[n]->w[l + 1] : (n == 0 ? a.oc.w[0] : a.P);
        if (p >= offs[n]->b[l] && p < bend) dst = nets[n]->gb[l] + (p - offs[n]->b[l]);
      }
    *dst = (float)s;
  }
  if (blockIdx.x == 0) {
    double tot[kMlpSums];
    for (int k = 0; k < kMlpSums; ++k) tot[k] = 0.0;
    for (long b = threadIdx.x; b < a.nblocks; b += kMlpBlock)
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
  long P, nblocks;
  size_t gpart, spart, total;
};

MlpLayout mlp_layout(long B, int D, int H, int A) {
  MlpLayout l;
  l.P = mlp_params(D, H, A) + mlp_params(D, H, 1);
  l.nblocks = (B + kMlpRows - 1) / kMlpRows;
  l.gpart = kHeaderBytes;
  l.spart = l.gpart + align_up((size_t)l.nblocks * l.P * sizeof(float), 256);
  l.total = l.spart + align_up((size_t)kMlpSums * l.nblocks * sizeof(double), 256);
  return l;
}

template <int H, int kAct>
const void* mlp_kernel_h(bool i64) {
  return i64 ? (const void*)mlp_cat_grad_kernel<H, kAct, int64_t>
             : (const void*)mlp_cat_grad_kernel<H, kAct, int32_t>;
}

template <int kAct>
const void* mlp_kernel_act(int H, bool i64) {
  switch (H) {
    case 16: return mlp_kernel_h<16, kAct>(i64);
    case 32: return mlp_kernel_h<32, kAct>(i64);
    case 64: return mlp_kernel_h<64, kAct>(i64);
    case 128: return mlp_kernel_h<128, kAct>(i64);
    default: return nullptr;
  }
}

bool mlp_net_ok(const ppo_mlp3_f32* n) {
  if (!n) return false;
  for (int l = 0; l < 3; ++l)
    if (!n->weight[l] || !n->bias[l] || !n->weight_grad[l] || !n->bias_grad[l]) return false;
  return true;
}

MlpNet to_net(const ppo_mlp3_f32* n) {
  MlpNet m;
  for (int l = 0; l < 3; ++l) {
    m.w[l] = n->weight[l];
    m.b[l] = n->bias[l];
    m.gw[l] = n->weight_grad[l];
    m.gb[l] = n->bias_grad[l];
  }
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
  if (B < 0 || n < 0) return PPO_ERR_INVALID_ARG;
  if (obs_dim <= 0 || obs_dim > kMlpMaxIn || A <= 0 || A > kMlpMaxA) return PPO_ERR_UNSUPPORTED;
  if (activation != PPO_ACT_RELU && activation != PPO_ACT_TANH) return PPO_ERR_INVALID_ARG;
  const void* kern = activation == PPO_ACT_TANH ? mlp_kernel_act<PPO_ACT_TANH>(hidden, actions_are_int64)
                                                : mlp_kernel_act<PPO_ACT_RELU>(hidden, actions_are_int64);
  if (!kern) return PPO_ERR_UNSUPPORTED;
  if (!mlp_net_ok(actor) || !mlp_net_ok(critic) || !params || !scalars_out)
    return PPO_ERR_INVALID_ARG;
  if (B == 0) return PPO_OK;
  if (!observations || !actions || !old_log_probs || !advantages || !returns)
    return PPO_ERR_INVALID_ARG;
  if (B > (1L << 31) || n > (1L << 40)) return PPO_ERR_TOO_LARGE;
  if (!workspace || workspace_bytes < ppo_mlp_cat_grad_workspace_bytes(B, obs_dim, hidden, A))
    return PPO_ERR_WORKSPACE;
  for (int l = 0; l < 3; ++l)
    if (!aligned(actor->weight[l], 16) || !aligned(critic->weight[l], 16))
      return PPO_ERR_INVALID_ARG;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  const MlpLayout l = mlp_layout(B, obs_dim, hidden, A);
  char* ws = static_cast<char*>(workspace);

  MlpArgs a = {};
  a.actor = to_net(actor);
  a.critic = to_net(critic);
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

  void* args[] = {&a};
  int st = hip_status(hipLaunchKernel(kern, dim3((unsigned)l.nblocks), dim3(kMlpBlock), args, 0,
                                      stream));
  if (st) return st;
  const long rblocks = (l.P + kMlpBlock - 1) / kMlpBlock;
  return hip_status(hipLaunchKernel((const void*)mlp_grad_reduce_kernel, dim3((unsigned)rblocks),
                                    dim3(kMlpBlock), args, 0, stream));
}
