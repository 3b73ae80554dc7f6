// Update-loop kernels around the fused loss (rl/deep/agents/ppo.py:129-171):
//
//  * ppo_gather_rows — the minibatch gather of ppo.py:132-139
//    (observations[batch_indices], actions[...], ...): every array's rows at
//    one index vector, in one launch instead of one torch gather per array.
//  * ppo_adam_clip_f32 — nn.utils.clip_grad_norm_(params, max_norm) followed
//    by torch.optim.Adam.step() (ppo.py:170-171), for up to
//    PPO_ADAM_MAX_TENSORS tensors in two launches: per-block sums of squared
//    gradients, then a pass in which every block derives the global norm and
//    the clip coefficient from those sums and updates its slice of
//    gradients, moments and parameters.  The fp32 arithmetic follows torch's
//    multi-tensor Adam op by op (lerp for the first moment, mul + addcmul for
//    the second, sqrt / bias-correction / eps / addcdiv for the update), each
//    operation rounded separately.
#include <algorithm>

#include "adam.hpp"
#include "common.hpp"

namespace ppo {
namespace {

// ---------------------------------------------------------------------------
// gather
// ---------------------------------------------------------------------------
struct GatherTable {
  const unsigned* src[PPO_GATHER_MAX_ARRAYS];
  unsigned* dst[PPO_GATHER_MAX_ARRAYS];
  int words[PPO_GATHER_MAX_ARRAYS];           // 4-byte words per row
  int word_start[PPO_GATHER_MAX_ARRAYS + 1];  // prefix of words over arrays
  int narr;
};

__global__ void __launch_bounds__(kBlock) gather_rows_kernel(GatherTable t,
                                                             const int64_t* __restrict__ idx,
                                                             long B, long nsrc) {
  const long W = t.word_start[t.narr];
  const long total = B * W;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long u = (long)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += stride) {
    const long b = u / W;
    const int w = (int)(u - b * W);
    int k = 0;
    while (k + 1 < t.narr && w >= t.word_start[k + 1]) ++k;
    const int ww = w - t.word_start[k];
    const long i = idx[b];
    unsigned val = 0u;  // rows for out-of-range indices are zero (no out-of-bounds read)
    if (i >= 0 && i < nsrc) val = t.src[k][i * t.words[k] + ww];
    t.dst[k][b * t.words[k] + ww] = val;
  }
}

// dst[i] = src[i] for i < n elements of T (src may be pinned host memory
// mapped into the device's address space; 16-byte elements when both ends
// are aligned, so each bus read carries four words).
template <typename T>
__global__ void __launch_bounds__(kBlock) copy_words_kernel(const T* __restrict__ src,
                                                            T* __restrict__ dst, long n) {
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = src[i];
}

// ---------------------------------------------------------------------------
// clip_grad_norm_ + Adam
// ---------------------------------------------------------------------------
constexpr int kAdamPerThread = 4;
constexpr long kAdamChunk = (long)kBlock * kAdamPerThread;  // elements per block
constexpr long kAdamLdsParts = 2048;  // sum-of-squares partials staged in LDS per round

struct AdamTable {
  float* p[PPO_ADAM_MAX_TENSORS];
  float* g[PPO_ADAM_MAX_TENSORS];
  float* m[PPO_ADAM_MAX_TENSORS];
  float* v[PPO_ADAM_MAX_TENSORS];
  long n[PPO_ADAM_MAX_TENSORS];
  long block_start[PPO_ADAM_MAX_TENSORS + 1];  // update blocks of each tensor
  long part_start[PPO_ADAM_MAX_TENSORS + 1];   // its sum-of-squares partials
  int nt;
};

__device__ __forceinline__ int tensor_of_block(const AdamTable& t, long b) {
  int k = 0;
  while (k + 1 < t.nt && b >= t.block_start[k + 1]) ++k;
  return k;
}

__global__ void __launch_bounds__(kBlock) adam_sumsq_kernel(AdamTable t, double* partial,
                                                            int64_t* step_counter) {
  const long b = blockIdx.x;
  if (step_counter && b == 0 && threadIdx.x == 0) *step_counter += 1;
  const int k = tensor_of_block(t, b);
  const long lo = (b - t.block_start[k]) * kAdamChunk;
  const long hi = lo + kAdamChunk < t.n[k] ? lo + kAdamChunk : t.n[k];
  double acc[1] = {0.0};
  for (long i = lo + threadIdx.x; i < hi; i += blockDim.x) {
    const double x = (double)t.g[k][i];
    acc[0] += x * x;
  }
  block_sum<1>(acc);
  if (threadIdx.x == 0) partial[b] = acc[0];
}

__global__ void __launch_bounds__(kBlock) adam_update_kernel(AdamTable t,
                                                             const double* __restrict__ partial,
                                                             AdamScalars s, float* norm_out,
                                                             const int64_t* step_counter) {
  __shared__ float s_coef;
  __shared__ float s_norm[PPO_ADAM_MAX_TENSORS];
  __shared__ double s_part[kAdamLdsParts];
  // The block's elements, moments and parameters are loaded first (they do
  // not depend on the norm), so their latency overlaps the norm's.
  const long b = blockIdx.x;
  const int k = tensor_of_block(t, b);
  const long lo = (b - t.block_start[k]) * kAdamChunk;
  const long hi = lo + kAdamChunk < t.n[k] ? lo + kAdamChunk : t.n[k];
  float* __restrict__ p = t.p[k];
  float* __restrict__ g = t.g[k];
  float* __restrict__ m = t.m[k];
  float* __restrict__ v = t.v[k];
  float gr[kAdamPerThread], mr[kAdamPerThread], vr[kAdamPerThread], pr[kAdamPerThread];
#pragma unroll
  for (int j = 0; j < kAdamPerThread; ++j) {
    const long i = lo + threadIdx.x + (long)j * kBlock;
    const long ic = i < hi ? i : lo;  // in range: lo < hi for every block
    gr[j] = g[ic];
    mr[j] = m[ic];
    vr[j] = v[ic];
    pr[j] = p[ic];
  }
  // Global norm: per-tensor norms rounded to fp32, then the norm of those in
  // tensor order (the two-level form of torch's _get_total_norm); every block
  // derives the same value in the same order.  The sum-of-squares partials
  // are staged in LDS by the whole block (their first round loaded with the
  // elements above), then wave w sums tensors w, w + 4, ...: lane l takes
  // partials l, l + 64, ... of the tensor and the wave's lanes are combined by
  // a fixed shuffle tree.
  constexpr int kPre = kAdamLdsParts / kBlock;
  const long total = t.part_start[t.nt];
  double pre[kPre];
#pragma unroll
  for (int q = 0; q < kPre; ++q) {
    const long i = threadIdx.x + (long)q * kBlock;
    pre[q] = i < total && i < kAdamLdsParts ? partial[i] : 0.0;
  }
  if (step_counter) adam_step_scalars_at(s, (double)*step_counter);
  const int lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  constexpr int kWavesA = kBlock / kWave;
  constexpr int kPerWave = (PPO_ADAM_MAX_TENSORS + kWavesA - 1) / kWavesA;
  double acc[kPerWave];
#pragma unroll
  for (int u = 0; u < kPerWave; ++u) acc[u] = 0.0;
  for (long base = 0; base < total; base += kAdamLdsParts) {
    const long cnt = total - base < kAdamLdsParts ? total - base : kAdamLdsParts;
    if (base == 0) {
#pragma unroll
      for (int q = 0; q < kPre; ++q) {
        const long i = threadIdx.x + (long)q * kBlock;
        if (i < cnt) s_part[i] = pre[q];
      }
    } else {
      for (long i = threadIdx.x; i < cnt; i += kBlock) s_part[i] = partial[base + i];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kPerWave; ++u) {
      const int kk = wv + u * kWavesA;
      if (kk < t.nt) {
        const long c0 = t.part_start[kk] > base ? t.part_start[kk] : base;
        const long c1 = t.part_start[kk + 1] < base + cnt ? t.part_start[kk + 1] : base + cnt;
        for (long c = c0 + lane; c < c1; c += kWave) acc[u] += s_part[c - base];
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < kPerWave; ++u) {
    const int kk = wv + u * kWavesA;
    const double sk = wave_sum(acc[u]);
    if (lane == 0 && kk < PPO_ADAM_MAX_TENSORS) s_norm[kk] = kk < t.nt ? (float)sqrt(sk) : 0.0f;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float norm;
    s_coef = adam_coef_from_norms(s, s_norm, t.nt, norm);
    if (blockIdx.x == 0 && norm_out) *norm_out = norm;
  }
  __syncthreads();
  const float coef = s_coef;
#pragma unroll
  for (int j = 0; j < kAdamPerThread; ++j) {
    const long i = lo + threadIdx.x + (long)j * kBlock;
    if (i >= hi) break;
    float gi, mi, vi, pi;
    adam_elem(s, coef, gr[j], mr[j], vr[j], pr[j], gi, mi, vi, pi);
    if (s.clip) g[i] = gi;
    p[i] = pi;
    m[i] = mi;
    v[i] = vi;
  }
}


long adam_blocks(int nt, const int64_t* numel, long* starts) {
  long b = 0;
  for (int k = 0; k < nt; ++k) {
    starts[k] = b;
    b += (numel[k] + kAdamChunk - 1) / kAdamChunk;
  }
  starts[nt] = b;
  return b;
}

}  // namespace

AdamScalars make_adam_scalars(const ppo_adam_params* hp) {
  const double step = hp->step_counter ? 1.0 : (double)hp->step;  // device path recomputes
  const double bc1 = 1.0 - pow(hp->beta1, step);
  const double bc2 = 1.0 - pow(hp->beta2, step);
  AdamScalars s;
  s.max_norm = (float)hp->max_grad_norm;
  s.clip = hp->max_grad_norm > 0.0 ? 1 : 0;
  s.beta1_w = (float)(1.0 - hp->beta1);
  s.beta2 = (float)hp->beta2;
  s.one_m_beta2 = (float)(1.0 - hp->beta2);
  s.bc2_sqrt = (float)sqrt(bc2);
  s.eps = (float)hp->eps;
  s.neg_step = (float)((hp->lr / bc1) * -1.0);
  s.lr_d = hp->lr;
  s.beta1_d = hp->beta1;
  s.beta2_d = hp->beta2;
  return s;
}

int launch_adam_presummed(int nt, float* const* params, float* const* grads,
                          float* const* exp_avg, float* const* exp_avg_sq, const int64_t* numel,
                          const ppo_adam_params* hp, const double* partials,
                          const long* part_start, float* grad_norm_out, hipStream_t stream) {
  if (nt < 1 || nt > PPO_ADAM_MAX_TENSORS || !hp) return PPO_ERR_INVALID_ARG;
  if ((!hp->step_counter && hp->step < 1) || !(hp->lr >= 0.0) || !(hp->eps >= 0.0))
    return PPO_ERR_INVALID_ARG;
  AdamTable t = {};
  t.nt = nt;
  for (int k = 0; k < nt; ++k) {
    t.p[k] = params[k];
    t.g[k] = grads[k];
    t.m[k] = exp_avg[k];
    t.v[k] = exp_avg_sq[k];
    t.n[k] = numel[k];
  }
  for (int k = 0; k <= nt; ++k) t.part_start[k] = part_start[k];
  const long blocks = adam_blocks(nt, numel, t.block_start);
  if (blocks == 0) return PPO_OK;
  if (blocks > 0x7fffffffL) return PPO_ERR_TOO_LARGE;
  hipLaunchKernelGGL(adam_update_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, stream, t,
                     partials, make_adam_scalars(hp), grad_norm_out, hp->step_counter);
  return last_launch_status();
}

}  // namespace ppo

extern "C" int ppo_gather_rows(const int64_t* index, int64_t B, int64_t n_src, int32_t narrays,
                               const void* const* src, const int32_t* row_bytes,
                               void* const* dst, void* stream_ptr) {
  using namespace ppo;
  if (B < 0 || n_src < 0 || narrays < 1 || narrays > PPO_GATHER_MAX_ARRAYS) return PPO_ERR_INVALID_ARG;
  if (B == 0) return PPO_OK;
  if (!index || !src || !row_bytes || !dst) return PPO_ERR_INVALID_ARG;
  GatherTable t = {};
  t.narr = narrays;
  long w = 0;
  for (int k = 0; k < narrays; ++k) {
    if (!src[k] || !dst[k] || row_bytes[k] <= 0 || row_bytes[k] % 4) return PPO_ERR_INVALID_ARG;
    t.src[k] = static_cast<const unsigned*>(src[k]);
    t.dst[k] = static_cast<unsigned*>(dst[k]);
    t.words[k] = row_bytes[k] / 4;
    t.word_start[k] = (int)w;
    w += t.words[k];
  }
  t.word_start[narrays] = (int)w;
  // word offsets are 32-bit in the kernel's table; B * w must not overflow
  if (w > (1L << 30) || B > (1L << 50) / w) return PPO_ERR_TOO_LARGE;
  const long total = (long)B * w;
  long blocks = std::min((total + kBlock - 1) / kBlock, 8192L);
  hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)blocks), dim3(kBlock), 0,
                     reinterpret_cast<hipStream_t>(stream_ptr), t, index, (long)B, (long)n_src);
  return last_launch_status();
}

extern "C" int ppo_copy_from_pinned(void* dst, const void* src_host, int64_t nbytes,
                                    void* stream_ptr) {
  using namespace ppo;
  if (nbytes < 0 || nbytes % 4 || nbytes >= (1L << 31)) return PPO_ERR_INVALID_ARG;
  if (nbytes == 0) return PPO_OK;
  if (!dst || !src_host) return PPO_ERR_INVALID_ARG;
  // the device's view of the pinned allocation; fails (and nothing is
  // launched) for memory the runtime did not pin and map
  void* src_dev = nullptr;
  hipError_t e = hipHostGetDevicePointer(&src_dev, const_cast<void*>(src_host), 0);
  if (e != hipSuccess || !src_dev) {
    (void)hipGetLastError();
    return PPO_ERR_INVALID_ARG;
  }
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  if (nbytes % 16 == 0 && aligned(src_dev, 16) && aligned(dst, 16)) {
    const long n = nbytes / 16;
    const long blocks = std::min((n + kBlock - 1) / kBlock, 1024L);
    hipLaunchKernelGGL(copy_words_kernel<uint4>, dim3((unsigned)blocks), dim3(kBlock), 0, stream,
                       static_cast<const uint4*>(src_dev), static_cast<uint4*>(dst), n);
  } else {
    const long n = nbytes / 4;
    const long blocks = std::min((n + kBlock - 1) / kBlock, 1024L);
    hipLaunchKernelGGL(copy_words_kernel<unsigned>, dim3((unsigned)blocks), dim3(kBlock), 0,
                       stream, static_cast<const unsigned*>(src_dev), static_cast<unsigned*>(dst),
                       n);
  }
  return last_launch_status();
}

extern "C" size_t ppo_adam_clip_workspace_bytes(int32_t ntensors, const int64_t* numel) {
  using namespace ppo;
  if (ntensors < 1 || ntensors > PPO_ADAM_MAX_TENSORS || !numel) return kHeaderBytes;
  long starts[PPO_ADAM_MAX_TENSORS + 1];
  const long blocks = adam_blocks(ntensors, numel, starts);
  return kHeaderBytes + align_up((size_t)std::max(blocks, 1L) * sizeof(double), 256);
}

extern "C" int ppo_adam_clip_f32(int32_t ntensors, float* const* params, float* const* grads,
                                 float* const* exp_avg, float* const* exp_avg_sq,
                                 const int64_t* numel, const ppo_adam_params* hp,
                                 float* grad_norm_out, void* workspace, size_t workspace_bytes,
                                 void* stream_ptr) {
  using namespace ppo;
  if (ntensors < 1 || ntensors > PPO_ADAM_MAX_TENSORS) return PPO_ERR_INVALID_ARG;
  if (!params || !grads || !exp_avg || !exp_avg_sq || !numel || !hp) return PPO_ERR_INVALID_ARG;
  if ((!hp->step_counter && hp->step < 1) || !(hp->lr >= 0.0) || !(hp->eps >= 0.0))
    return PPO_ERR_INVALID_ARG;
  for (int k = 0; k < ntensors; ++k)
    if (numel[k] < 0) return PPO_ERR_INVALID_ARG;
  if (!workspace || workspace_bytes < ppo_adam_clip_workspace_bytes(ntensors, numel))
    return PPO_ERR_WORKSPACE;
  AdamTable t = {};
  t.nt = ntensors;
  for (int k = 0; k < ntensors; ++k) {
    if (numel[k] < 0) return PPO_ERR_INVALID_ARG;
    if (numel[k] > 0 && (!params[k] || !grads[k] || !exp_avg[k] || !exp_avg_sq[k]))
      return PPO_ERR_INVALID_ARG;
    t.p[k] = params[k];
    t.g[k] = grads[k];
    t.m[k] = exp_avg[k];
    t.v[k] = exp_avg_sq[k];
    t.n[k] = numel[k];
  }
  const long blocks = adam_blocks(ntensors, numel, t.block_start);
  if (blocks == 0) return PPO_OK;
  if (blocks > 0x7fffffffL) return PPO_ERR_TOO_LARGE;
  for (int k = 0; k <= ntensors; ++k) t.part_start[k] = t.block_start[k];
  const AdamScalars s = make_adam_scalars(hp);
  double* partial = reinterpret_cast<double*>(static_cast<char*>(workspace) + kHeaderBytes);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  hipLaunchKernelGGL(adam_sumsq_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, stream, t,
                     partial, hp->step_counter);
  int st = last_launch_status();
  if (st) return st;
  hipLaunchKernelGGL(adam_update_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, stream, t,
                     partial, s, grad_norm_out, hp->step_counter);
  return last_launch_status();
}
