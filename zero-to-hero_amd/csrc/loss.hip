// Fused PPO loss: forward scalars and backward gradients in one pass.
//
// Reference: PPOAgent._update_batch, rl/deep/agents/ppo.py:149-169.  The
// forward is
//     dist    = Categorical(logits=logits)                        (:150)
//     lp      = dist.log_prob(actions)                             (:151)
//     ratio   = exp(lp - old_log_probs)                            (:154)
//     clipped = ratio.clamp(1 - clip, 1 + clip)                    (:155-158)
//     policy  = -minimum(ratio * adv, clipped * adv)               (:159)
//     value   = mse_loss(values, returns)                          (:160)
//     loss    = policy.mean() + vc * value - ec * dist.entropy().mean()  (:163-167)
// and loss.backward() (:169) is replaced, down to the logits and the value
// head, by the closed-form gradient written directly (B rows, p = softmax):
//     g_lp      = -(adv/B) * ratio * (s_u + s_w * [lo <= ratio <= hi])
//                 with s_u/s_w the torch.minimum tie weights (1, 0, or 1/2)
//     dlogit_k  = g_lp * (1[k == a] - p_k) + (ec/B) * p_k * (log p_k + H)
//     dvalue    = vc * 2 * (v - R) / B          (or the clipped-value form)
// Gaussian variant: Normal(mu, exp(log_std)) summed over the action dims.
//
// Layout: one thread per row.  A workgroup walks 256-row tiles of the
// [B,A] logits (each tile a contiguous block of 256*A floats) on a grid
// capped at a few workgroups per CU; per tile it prefetches the per-row
// inputs into registers, stages the logits through LDS with float4 loads
// (row stride padded to an odd number of words, so the row-per-thread LDS
// reads are bank-conflict-free), and writes dlogits back through the same
// tile.  Loss scalars are summed per workgroup in fp64 and combined in a fixed
// order by a one-block finaliser kernel (deterministic, no float atomics).
#include <float.h>

#include <algorithm>

#include "common.hpp"
#include "grid_sync.hpp"
#include "row_math.hpp"

namespace ppo {
namespace {

// Widths handled by the row-per-thread kernels, chosen so that the LDS tiles
// (256 rows x odd-padded width, one tile for logits, two for mu/actions) plus
// the static reduction arrays stay under the 64 KiB a workgroup may address.
constexpr int kMaxCatRowWidth = 48;  // A above this uses the wave-per-row kernel
constexpr int kMaxGaussDim = 24;     // D limit of the Gaussian kernel
constexpr int kScalarSlots = 8;      // per-block partial doubles reserved for the loss scalars
constexpr int kGaussSlots = kScalarSlots + kMaxGaussDim;
constexpr long kWaveRowBlocks = 4096;  // grid cap of the wave-per-row kernel
#ifndef PPO_LOSS_BLOCKS_PER_CU
#define PPO_LOSS_BLOCKS_PER_CU 8
#endif
constexpr long kLossGridCap = 256L * PPO_LOSS_BLOCKS_PER_CU;  // 256 CUs on MI355X

struct LossArgs {
  const float* x;        // logits [B,A] or mu [B,D]
  const float* log_std;  // [D] (Gaussian)
  long B;
  int A;                 // A or D
  const void* actions;   // int32/int64 [B] or float [B,D]
  const float* old_lp;
  const float* adv;
  const float* ret;
  const float* val;
  const float* old_val;
  float lo, hi, clip;    // ratio clamp bounds and the clip parameter
  float vclip;
  int use_vclip;
  float vc, ec;          // value / entropy coefficients as fp32 (torch scalar math)
  float inv_b;
  float* dx;
  float* dlog_std;
  float* dval;
  float* scalars;
  double* partial;
  uint64_t* epoch;  // Gaussian: the workspace header's call counter
  int tag_slot;     // Gaussian: partial slot holding each workgroup's arrival tag
  int finish;       // Gaussian: 1 = collect in-kernel, 0 = loss_gauss_finish_kernel does
  int nopoll;       // the collection follows the loss launch: read the partials without polling
  int collector;    // wave-tile kernels: workgroups 0 .. collector-1 only collect (no tiles)
  WaitCtl wc;       // Gaussian in-kernel finish: poll limit, the device's wait-status word
};

// Streamed arrays are touched once: nontemporal loads/stores keep them from
// displacing reusable lines (measured on MI355X: a float4 copy goes from 5.5
// to 6.3 TB/s with nontemporal accesses and 4 loads in flight per thread).
// Ordinary stores make this kernel look faster in isolation (the north-star
// loss 268 -> 241 us after a read-only cache flush) but leave ~0.6 GB of
// dirty lines whose write-back lands in the next kernel: in the GAE + loss
// step the GAE call went from 53 to 69 us and the step from 305 to 333 us.
typedef float f4 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ T ldnt(const T* p) { return __builtin_nontemporal_load(p); }
template <typename T>
__device__ __forceinline__ void stnt(T v, T* p) { __builtin_nontemporal_store(v, p); }

// Per-row inputs other than the logits/mu are loaded ahead of the LDS barrier.
__device__ __forceinline__ RowIn load_row(const LossArgs& a, long row) {
  RowIn r;
  r.old_lp = ldnt(a.old_lp + row);
  r.adv = ldnt(a.adv + row);
  r.ret = ldnt(a.ret + row);
  r.v = ldnt(a.val + row);
  r.vo = a.use_vclip ? ldnt(a.old_val + row) : 0.0f;
  return r;
}

// Everything per row that does not depend on the policy family (row_math.hpp);
// stores dvalue.
__device__ __forceinline__ RowOut ppo_row(const LossArgs& a, long row, const RowIn& in,
                                          float lp) {
  const RowOut o = ppo_row_math(a, in, lp);
  stnt(o.dval, a.dval + row);
  return o;
}

// Row index of flat element e in a tile of `width`-float rows, without an
// integer divide: e <= 256*64, so (e + 0.5) * (1/width) is never within
// rounding distance of an integer boundary.
__device__ __forceinline__ int row_of(int e, float inv_width) {
  return (int)(((float)e + 0.5f) * inv_width);
}

// Copy `count` floats from global (contiguous) into an LDS tile of row
// stride `ws` (count = rows * width).
template <bool kVec>
__device__ __forceinline__ void stage_in(const float* src, int count, int width, float inv_width,
                                         int ws, float* lds) {
  int start = 0;
  if constexpr (kVec) {
    const int n4 = count >> 2;
    const float4* s4 = reinterpret_cast<const float4*>(src);
    for (int i = threadIdx.x; i < n4; i += blockDim.x) {
      const float4 x = s4[i];
      const int e = i << 2;
      int r = row_of(e, inv_width);
      int c = e - r * width;
      const float xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        lds[r * ws + c] = xs[k];
        if (++c == width) { c = 0; ++r; }
      }
    }
    start = n4 << 2;
  }
  for (int e = start + threadIdx.x; e < count; e += blockDim.x) {
    const int r = row_of(e, inv_width);
    lds[r * ws + (e - r * width)] = src[e];
  }
}

template <bool kVec>
__device__ __forceinline__ void stage_out(float* dst, int count, int width, float inv_width,
                                          int ws, const float* lds) {
  int start = 0;
  if constexpr (kVec) {
    const int n4 = count >> 2;
    float4* d4 = reinterpret_cast<float4*>(dst);
    for (int i = threadIdx.x; i < n4; i += blockDim.x) {
      const int e = i << 2;
      int r = row_of(e, inv_width);
      int c = e - r * width;
      float xs[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        xs[k] = lds[r * ws + c];
        if (++c == width) { c = 0; ++r; }
      }
      d4[i] = make_float4(xs[0], xs[1], xs[2], xs[3]);
    }
    start = n4 << 2;
  }
  for (int e = start + threadIdx.x; e < count; e += blockDim.x) {
    const int r = row_of(e, inv_width);
    dst[e] = lds[r * ws + (e - r * width)];
  }
}

// Per-block partials are stored slot-major, partial[slot * gridDim.x + block]
// (slots 0-4: the loss sums; slots 5..5+D-1: the Gaussian dlog_std column
// sums), so the finaliser's loads of one slot are contiguous.
constexpr int kLossSums = 5;
static_assert(kLossSums + kMaxGaussDim < kGaussSlots,
              "the Gaussian arrival tag takes the last partial slot");

__device__ inline void store_partial(const LossArgs& a, int slot, double v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(a.partial) + (long)slot * gridDim.x + blockIdx.x,
                     __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block partial of the 5 loss sums.
__device__ inline void store_scalar_partials(const LossArgs& a, double (&acc)[5]) {
  block_sum<5>(acc);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int k = 0; k < 5; ++k) store_partial(a, k, acc[k]);
  }
}

__device__ __forceinline__ void accumulate(double (&acc)[5], const RowOut& o, float ent) {
  acc[0] += (double)o.pol;
  acc[1] += (double)o.vl;
  acc[2] += (double)ent;
  acc[3] += (double)o.kl;
  acc[4] += (double)o.clipped;
}

// One-block finaliser of the categorical loss, launched after the loss kernel
// on the same stream: sums the per-block partials in a fixed order (thread t
// takes blocks t, t + kFinalBlock, ...; then the block tree), so results are
// deterministic, and forms the means and the total loss.  The categorical
// and Gaussian kernels normally finish in-kernel (loss_publish below; see
// cat_finish_in_kernel for when the categorical loss does); this launch is
// the route without in-kernel waits.  Measured on MI355X: the in-kernel
// finish takes the Gaussian loss of B = 2,097,152, D = 6 from 49.0 to 45.2 us.
__global__ void __launch_bounds__(kFinalBlock) loss_finalize_kernel(LossArgs a, long nblocks) {
  constexpr int K = kLossSums;
  double tot[K];
#pragma unroll
  for (int k = 0; k < K; ++k) tot[k] = 0.0;
  // two blocks per thread per round, all loads in flight together (a block
  // past the grid re-reads block b0 and is masked out)
  for (long b0 = threadIdx.x; b0 < nblocks; b0 += 2 * kFinalBlock) {
    double v[2][K];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const long b = b0 + h * kFinalBlock < nblocks ? b0 + h * kFinalBlock : b0;
#pragma unroll
      for (int k = 0; k < K; ++k) v[h][k] = a.partial[(long)k * nblocks + b];
    }
    const bool second = b0 + kFinalBlock < nblocks;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int k = 0; k < K; ++k) tot[k] += (h == 0 || second) ? v[h][k] : 0.0;
  }
  block_sum<K>(tot);
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

// The finish of the Gaussian loss kernels, after their partials are stored: each
// workgroup waits until its partial stores are complete and then stores its
// arrival tag.  Collector workgroups (every workgroup of the grid is resident:
// the host sizes it by occupancy) then wait (bounded) for every tag of this
// call and sum one group of partial slots each, in a fixed order (thread t
// takes blocks t, t + kBlock, ...; then the block tree), so results are
// deterministic: group 0, the five loss sums, in workgroup 0, which forms the
// means and the total loss; group 1 + d, the Gaussian dlog_std column d, in
// workgroup 1 + d (wrapping around the grid), which writes
// dlog_std[d] = sum over blocks - ec.  The tag of a call is a hash of the
// workspace's call counter, which workgroup 0 advances at the end: a tag left
// by an earlier call (or graph replay) never matches, and no word needs
// clearing.  No atomic read-modify-write is involved, so arrivals do not
// serialise on one address; a wait that gives up leaves NaN results.
__device__ __forceinline__ uint64_t loss_tag(uint64_t epoch) {
  return (epoch * 0x9E3779B97F4A7C15ULL) ^ kSlotTag;
}

// Sums slots slot0..slot0+K-1 over all blocks once their tags read `tag`
// (K = 5: the loss sums; K = 1: one dlog_std column); the totals end in
// every lane of wave 0.
template <int K>
__device__ void collect_slots(const LossArgs& a, long nb, int slot0, uint64_t tag,
                              double (&tot)[K]) {
  constexpr int kPer = 4;  // blocks a thread polls and loads together
  const uint64_t* part = reinterpret_cast<const uint64_t*>(a.partial);
  const uint64_t* tags = part + (long)a.tag_slot * nb;
#pragma unroll
  for (int k = 0; k < K; ++k) tot[k] = 0.0;
  bool ok = true;
  for (long b0 = threadIdx.x; b0 < nb; b0 += kPer * kBlock) {
    for (long it = 0; !a.nopoll; ++it) {
      if (it >= a.wc.spin) {
        ok = false;
        break;
      }
      uint64_t w[kPer];
#pragma unroll
      for (int h = 0; h < kPer; ++h) {
        const long b = b0 + h * kBlock < nb ? b0 + h * kBlock : b0;
        w[h] = __hip_atomic_load(tags + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      bool all = true;
#pragma unroll
      for (int h = 0; h < kPer; ++h) all = all && w[h] == tag;
      if (all) break;
      __builtin_amdgcn_s_sleep(1);
    }
    // every load issued before any is consumed (blocks past the grid
    // re-read block b0, masked out below)
    double v[kPer][K];
#pragma unroll
    for (int h = 0; h < kPer; ++h) {
      const long b = b0 + h * kBlock < nb ? b0 + h * kBlock : b0;
#pragma unroll
      for (int k = 0; k < K; ++k)
        v[h][k] = __builtin_bit_cast(double, __hip_atomic_load(part + (long)(slot0 + k) * nb + b,
                                                               __ATOMIC_RELAXED,
                                                               __HIP_MEMORY_SCOPE_AGENT));
    }
#pragma unroll
    for (int h = 0; h < kPer; ++h)
#pragma unroll
      for (int k = 0; k < K; ++k) tot[k] += b0 + h * kBlock < nb ? v[h][k] : 0.0;
  }
  if (!ok) {
#pragma unroll
    for (int k = 0; k < K; ++k) tot[k] = __builtin_nan("");
    wait_report(a.wc.status);
  }
  block_sum<K>(tot);
}

// Collector `b` of `ncoll` sums the slot groups it owns over the `nb`
// publishing workgroups, all tagged loss_tag(epn): groups 1 + d (dlog_std
// column d) go round-robin from collector 1, and collector 0 takes the
// groups left over and then group 0, the loss sums, forms the scalars and
// stores epn as the call counter.
template <int MAXD>
__device__ void loss_collect(const LossArgs& a, long nb, uint64_t epn, long b, long ncoll) {
  __shared__ float s_hterm[MAXD > 0 ? MAXD : 1];
  const int tid = threadIdx.x;
  const int D = MAXD > 0 ? a.A : 0;
  if (b > (long)D) return;  // no slot group here
  if (b == 0 && MAXD > 0 && tid < D) {
    // Gaussian entropy term per dim, summed in dim order below
    const float kEntConst = 1.41893853320467274178f;  // 0.5 + 0.5*log(2*pi)
    s_hterm[tid] = kEntConst + logf(expf(a.log_std[tid]));
  }
  __syncthreads();
  const uint64_t tag = loss_tag(epn);
  if (MAXD > 0) {
    for (long grp = b + (b == 0 ? ncoll : 0); grp <= D; grp += ncoll) {
      if (grp == 0) continue;
      double col[1];
      collect_slots<1>(a, nb, kLossSums + (int)grp - 1, tag, col);
      if (tid == 0) a.dlog_std[grp - 1] = (float)col[0] - a.ec;
    }
  }
  if (b != 0) return;
  double tot[kLossSums];
  collect_slots<kLossSums>(a, nb, 0, tag, tot);
  if (tid == 0) {
    float ent;
    if (MAXD > 0) {
      // entropy of Normal(mu, scale) summed over dims, identical for every row
      float h = 0.0f;
      for (int d = 0; d < D; ++d) h += s_hterm[d];
      ent = h;
    } else {
      ent = (float)(tot[2] / (double)a.B);
    }
    const double nbr = (double)a.B;
    const float pol = (float)(tot[0] / nbr);
    const float vl = (float)(tot[1] / nbr);
    a.scalars[PPO_SCALAR_POLICY] = pol;
    a.scalars[PPO_SCALAR_VALUE] = vl;
    a.scalars[PPO_SCALAR_ENTROPY] = ent;
    a.scalars[PPO_SCALAR_APPROX_KL] = (float)(tot[3] / nbr);
    a.scalars[PPO_SCALAR_CLIPFRAC] = (float)(tot[4] / nbr);
    a.scalars[PPO_SCALAR_LOSS] = (pol + a.vc * vl) - a.ec * ent;
    __hip_atomic_store(a.epoch, epn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int MAXD>
__device__ void loss_publish(const LossArgs& a) {
  __shared__ uint64_t s_ep;
  const int tid = threadIdx.x;
  const long nb = gridDim.x;
  uint64_t ep = 0;
  if (tid == 0) ep = __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the partial stores are complete
  __syncthreads();
  if (tid == 0) {
    uint64_t* tags = reinterpret_cast<uint64_t*>(a.partial) + (long)a.tag_slot * nb;
    __hip_atomic_store(tags + blockIdx.x, loss_tag(ep + 1), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    s_ep = ep + 1;
  }
  if (!a.finish) return;  // (loss_gauss_finish_kernel collects after the launch)
  __syncthreads();
  loss_collect<MAXD>(a, nb, s_ep, blockIdx.x, nb);
}

// The Gaussian finish as a launch of its own (no in-kernel wait: for grids
// whose co-residency the host could not establish, or PPO_AMD_GAUSS_FINISH=0):
// workgroup g sums slot group g of the `nb` workgroups of the loss launch
// before it, in the in-kernel collectors' order (same results bit for bit),
// reading the partials without polling their tags (the launch boundary
// orders them); workgroup 0 then forms the scalars and advances the call
// counter past the tags that launch stored.
template <int MAXD>
__global__ void __launch_bounds__(kBlock) loss_gauss_finish_kernel(LossArgs a, long nb) {
  __shared__ uint64_t s_ep;
  if (threadIdx.x == 0)
    s_ep = __hip_atomic_load(a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
  __syncthreads();
  a.nopoll = 1;
  loss_collect<MAXD>(a, nb, s_ep, blockIdx.x, gridDim.x);
}

// Action index of a row, or -1 when it lies outside [0, A).
template <typename ActT>
__device__ __forceinline__ int action_index(const LossArgs& a, ActT raw) {
  const long act = (long)raw;
  return (act >= 0 && act < a.A) ? (int)act : -1;
}

template <typename ActT>
__device__ __forceinline__ int row_action(const LossArgs& a, long row) {
  return action_index<ActT>(a, reinterpret_cast<const ActT*>(a.actions)[row]);
}

// The raw action of a row, loaded without inspecting it: a prefetch that
// validated it on the spot would make the compiler wait for every load in
// flight, the prefetched tile included.
template <typename ActT>
__device__ __forceinline__ ActT row_action_raw(const LossArgs& a, long row) {
  return __builtin_nontemporal_load(reinterpret_cast<const ActT*>(a.actions) + row);
}

// ---------------------------------------------------------------------------
// Categorical, A <= kMaxCatRowWidth: one thread per row, logits staged
// through LDS.  Softmax statistics in two passes over the row:
//   m = max z;  s = sum e_j, e_j = exp(z_j - m);  S = sum e_j (z_j - m)
//   log p_j = (z_j - m) - log s;   H = log s - S / s
// and a third pass recomputes e_j for the gradient (2 exp per logit).  The
// per-logit exponentials use the hardware exp2 (__expf: one multiply by
// log2(e) and v_exp_f32, relative error ~1e-6 for |z_j - m| <= 20); the
// accurate expf sequence costs ~10 VALU ops and made this kernel VALU-bound.
// The ratio exp(lp - old_lp) keeps the accurate expf.
// ---------------------------------------------------------------------------
template <typename ActT, bool kVec>
__global__ void __launch_bounds__(kBlock) loss_cat_kernel(LossArgs a, long ntiles) {
  extern __shared__ float s_tile[];
  const int A = a.A;
  const int AS = A | 1;
  const float invA = 1.0f / (float)A;
  const float ge = a.ec * a.inv_b;
  const int tid = threadIdx.x;
  double acc[5] = {0, 0, 0, 0, 0};

  for (long tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const long row0 = tile * kBlock;
    const int nrows = (int)std::min<long>(kBlock, a.B - row0);
    const long row = row0 + tid;
    RowIn in = {0, 0, 0, 0, 0};
    int ai = -1;
    if (tid < nrows) {
      in = load_row(a, row);
      ai = row_action<ActT>(a, row);
    }
    stage_in<kVec>(a.x + row0 * A, nrows * A, A, invA, AS, s_tile);
    __syncthreads();

    if (tid < nrows) {
      float* z = s_tile + tid * AS;
      float m = -INFINITY;
      for (int j = 0; j < A; ++j) m = fmaxf(m, z[j]);
      float s = 0.0f, S = 0.0f;
      for (int j = 0; j < A; ++j) {
        const float t = z[j] - m;
        const float e = __expf(t);
        s += e;
        S += e > 0.0f ? e * t : 0.0f;
      }
      const float log_s = logf(s);
      const float inv_s = 1.0f / s;
      const float H = log_s - S * inv_s;
      const float lp = ai >= 0 ? (z[ai] - m) - log_s : __builtin_nanf("");
      const RowOut o = ppo_row(a, row, in, lp);
      for (int j = 0; j < A; ++j) {
        const float t = z[j] - m;
        const float p = __expf(t) * inv_s;
        const float logp = fmaxf(t - log_s, -FLT_MAX);
        const float onehot = j == ai ? 1.0f : 0.0f;
        z[j] = o.g_lp * (onehot - p) + ge * (p * (logp + H));
      }
      accumulate(acc, o, H);
    }
    __syncthreads();
    stage_out<kVec>(a.dx + row0 * A, nrows * A, A, invA, AS, s_tile);
    __syncthreads();
  }
  store_scalar_partials(a, acc);
  if (a.finish) loss_publish<0>(a);
}

// ---------------------------------------------------------------------------
// Categorical, A <= 4*PF: the same per-row math as loss_cat_kernel,
// software-pipelined for 16-byte-aligned inputs.  Each
// thread holds up to PF float4 of the next tile's logits plus its row
// inputs in registers: while tile i is computed out of LDS, the loads of
// tile i+1 are already in flight, so a workgroup never waits on HBM between
// tiles.  All streamed accesses are nontemporal.
// ---------------------------------------------------------------------------
template <typename ActT, int PF>
struct CatPrefetch {
  f4 x[PF];
  float tail;   // element n4*4 + tid of a tile whose size is not a multiple of 4
  RowIn in;
  ActT act;     // raw action (validated when the tile is processed)
  int nrows;
};

template <typename ActT, int PF>
__device__ __forceinline__ void cat_prefetch(const LossArgs& a, long tile, CatPrefetch<ActT, PF>& p) {
  const int tid = threadIdx.x;
  const long row0 = tile * kBlock;
  p.nrows = (int)std::min<long>(kBlock, a.B - row0);
  const int count = p.nrows * a.A;
  const int n4 = count >> 2;
  const f4* src = reinterpret_cast<const f4*>(a.x + row0 * a.A);
#pragma unroll
  for (int k = 0; k < PF; ++k) {
    const int i = k * kBlock + tid;
    if (i < n4) p.x[k] = ldnt(src + i);
  }
  if (tid < count - (n4 << 2)) p.tail = ldnt(a.x + row0 * a.A + (n4 << 2) + tid);
  if (tid < p.nrows) {
    const long row = row0 + tid;
    p.in = load_row(a, row);
    p.act = row_action_raw<ActT>(a, row);
  }
}

template <typename ActT, int PF>
__global__ void __launch_bounds__(kBlock) loss_cat_pipe_kernel(LossArgs a, long ntiles) {
  extern __shared__ float s_tile[];
  const int A = a.A;
  const int AS = A | 1;
  const float invA = 1.0f / (float)A;
  const float ge = a.ec * a.inv_b;
  const int tid = threadIdx.x;
  double acc[5] = {0, 0, 0, 0, 0};
  CatPrefetch<ActT, PF> pf;
  long tile = blockIdx.x;
  if (tile < ntiles) cat_prefetch<ActT, PF>(a, tile, pf);

  for (; tile < ntiles; tile += gridDim.x) {
    // registers -> LDS for the current tile
    const int nrows = pf.nrows;
    const int count = nrows * A;
    const int n4 = count >> 2;
#pragma unroll
    for (int k = 0; k < PF; ++k) {
      const int i = k * kBlock + tid;
      if (i < n4) {
        const int e = i << 2;
        int r = row_of(e, invA);
        int c = e - r * A;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          s_tile[r * AS + c] = pf.x[k][q];
          if (++c == A) { c = 0; ++r; }
        }
      }
    }
    if (tid < count - (n4 << 2)) {
      const int e = (n4 << 2) + tid;
      const int r = row_of(e, invA);
      s_tile[r * AS + (e - r * A)] = pf.tail;
    }
    const RowIn in = pf.in;
    const int ai = tid < nrows ? action_index<ActT>(a, pf.act) : -1;
    const long row0 = tile * kBlock;
    __syncthreads();

    // next tile's loads go out before this tile's math
    const long next = tile + gridDim.x;
    if (next < ntiles) cat_prefetch<ActT, PF>(a, next, pf);

    if (tid < nrows) {
      const long row = row0 + tid;
      float* z = s_tile + tid * AS;
      float m = -INFINITY;
      for (int j = 0; j < A; ++j) m = fmaxf(m, z[j]);
      float s = 0.0f, S = 0.0f;
      for (int j = 0; j < A; ++j) {
        const float t = z[j] - m;
        const float e = __expf(t);
        s += e;
        S += e > 0.0f ? e * t : 0.0f;
      }
      const float log_s = logf(s);
      const float inv_s = 1.0f / s;
      const float H = log_s - S * inv_s;
      const float lp = ai >= 0 ? (z[ai] - m) - log_s : __builtin_nanf("");
      const RowOut o = ppo_row(a, row, in, lp);
      for (int j = 0; j < A; ++j) {
        const float t = z[j] - m;
        const float p = __expf(t) * inv_s;
        const float logp = fmaxf(t - log_s, -FLT_MAX);
        const float onehot = j == ai ? 1.0f : 0.0f;
        z[j] = o.g_lp * (onehot - p) + ge * (p * (logp + H));
      }
      accumulate(acc, o, H);
    }
    __syncthreads();
    // LDS -> dlogits, nontemporal float4 stores
    f4* dst = reinterpret_cast<f4*>(a.dx + row0 * A);
    for (int i = tid; i < n4; i += kBlock) {
      const int e = i << 2;
      int r = row_of(e, invA);
      int c = e - r * A;
      f4 v;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[q] = s_tile[r * AS + c];
        if (++c == A) { c = 0; ++r; }
      }
      stnt(v, dst + i);
    }
    if (tid < count - (n4 << 2)) {
      const int e = (n4 << 2) + tid;
      const int r = row_of(e, invA);
      a.dx[row0 * A + e] = s_tile[r * AS + (e - r * A)];
    }
    __syncthreads();
  }
  store_scalar_partials(a, acc);
  if (a.finish) loss_publish<0>(a);
}

// ---------------------------------------------------------------------------
// Categorical, A <= MAXA and A % 4 != 0, 16-byte-aligned inputs: wave tiles,
// the register-resident form.  Each wave owns a tile of 64 consecutive rows
// (one contiguous span of 64*A floats, 16*A float4) and stages it through its
// own slice of LDS in its global layout (one ds_write_b128 / ds_read_b128 per
// float4, no index arithmetic), so the transposition between the coalesced
// float4 layout and one-row-per-lane needs no workgroup barrier: a wave's LDS
// operations execute in issue order, and a wave-level compiler barrier keeps
// the compiler from moving LDS accesses across the hand-offs.  Waves stream
// independently, each with the next tile's loads in flight during the
// current tile's math.  Each lane reads its row into registers once and
// evaluates, per logit,
//     t_j = max(z_j - m, -FLT_MAX),  e_j = exp(t_j),  s += e_j,  S += e_j t_j
//     dlogit_j = (e_j / s) * (ec/B * t_j + K),  K = ec/B * (H - log s) - g_lp
// which is the gradient of the LDS-pass form rearranged (log p_j = t_j -
// log s); the 1[j == a] * g_lp term is added by one LDS read-modify-write per
// row.  That is ~10 VALU operations per logit against ~40 for the LDS-pass
// form, which was VALU-bound on MI355X.  KA > 0 fixes A at compile time (no
// per-logit predicates); KA == 0 takes A from the arguments, A <= MAXA.
//
// Full tiles run branch-free: lane l moves float4 min(64k + l, 16A - 1) for
// k < ceil(A/4) (lanes past the end repeat the last float4: same address,
// same value), the action is validated only when used, and vf_clip is a
// template parameter.  With no data-dependent branch between a tile's
// prefetch and the next tile's staging, the compiler waits only for the
// prefetched loads there, not for the previous tile's stores (on gfx9 the
// vector memory counter counts stores too).  The last, partial tile
// (B mod 64 rows) is processed after the loop with predicated accesses.
// ---------------------------------------------------------------------------
template <bool kVclip>
__device__ __forceinline__ RowIn load_row_t(const LossArgs& a, long row) {
  RowIn r;
  r.old_lp = ldnt(a.old_lp + row);
  r.adv = ldnt(a.adv + row);
  r.ret = ldnt(a.ret + row);
  r.v = ldnt(a.val + row);
  r.vo = kVclip ? ldnt(a.old_val + row) : 0.0f;
  return r;
}

template <typename ActT, int PF>
struct WavePrefetch {
  f4 x[PF];
  RowIn in;
  ActT act;  // raw action (validated when the tile is processed)
};

template <typename ActT, int PF, bool kVclip>
__device__ __forceinline__ void wave_prefetch(const LossArgs& a, long wt, int lane, int n4,
                                              WavePrefetch<ActT, PF>& p) {
  const long row0 = wt * kWave;
  const f4* src = reinterpret_cast<const f4*>(a.x + row0 * a.A);
#pragma unroll
  for (int k = 0; k < PF; ++k) p.x[k] = ldnt(src + std::min(k * kWave + lane, n4 - 1));
  // keep the logits loads ahead of the row loads in every copy of this
  // prefetch, so the staging wait can leave the row loads (and any later
  // stores) outstanding on every path into the loop
  __builtin_amdgcn_sched_barrier(0);
  p.in = load_row_t<kVclip>(a, row0 + lane);
  p.act = row_action_raw<ActT>(a, row0 + lane);
}

// Orders this wave's LDS accesses before and after a cross-lane hand-off.
__device__ __forceinline__ void wave_lds_handoff() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One row from LDS (zr: A logits) to its gradient in place; accumulates the
// row's loss terms (the formulas above).
template <int KA, int MAXA>
__device__ __forceinline__ void cat_row_math(const LossArgs& a, float* zr, int A, long row,
                                             const RowIn& in, int ai, float ge,
                                             double (&acc)[5]) {
  float H;
  const RowOut o = cat_row_grad<MAXA>(a, zr, A, ai, ge, in, H);
  stnt(o.dval, a.dval + row);
  accumulate(acc, o, H);
}

template <typename ActT, int KA, int MAXA, bool kVclip>
__global__ void __launch_bounds__(kBlock) loss_cat_wtile_kernel(LossArgs a, long nfull) {
  constexpr int PF = (MAXA + 3) / 4;
  constexpr int kWavesPerBlock = kBlock / kWave;
  extern __shared__ float s_lds[];
  const int A = KA > 0 ? KA : a.A;
  const int n4 = (kWave / 4) * A;  // float4 per full tile
  const float ge = a.ec * a.inv_b;
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  float* s_tile = s_lds + wid * kWave * A;  // 256*A bytes: 16-byte aligned
  f4* s_tile4 = reinterpret_cast<f4*>(s_tile);
  double acc[5] = {0, 0, 0, 0, 0};
  WavePrefetch<ActT, PF> pf;
  // (with a.collector, workgroup 0 takes no tiles: it only collects the others' partials)
  const long c0 = a.collector;
  const long wstride = ((long)gridDim.x - c0) * kWavesPerBlock;
  long wt = (long)blockIdx.x < c0 ? nfull + 1 : ((long)blockIdx.x - c0) * kWavesPerBlock + wid;
  if (wt < nfull) wave_prefetch<ActT, PF, kVclip>(a, wt, lane, n4, pf);

  for (; wt < nfull; wt += wstride) {
#pragma unroll
    for (int k = 0; k < PF; ++k) s_tile4[std::min(k * kWave + lane, n4 - 1)] = pf.x[k];
    const RowIn in = pf.in;
    const int ai = action_index<ActT>(a, pf.act);
    const long row0 = wt * kWave;
    wave_lds_handoff();

    const long next = wt + wstride;
    if (next < nfull) wave_prefetch<ActT, PF, kVclip>(a, next, lane, n4, pf);

    cat_row_math<KA, MAXA>(a, s_tile + lane * A, A, row0 + lane, in, ai, ge, acc);
    wave_lds_handoff();
    f4* dst = reinterpret_cast<f4*>(a.dx + row0 * A);
#pragma unroll
    for (int k = 0; k < PF; ++k) {
      const int i = std::min(k * kWave + lane, n4 - 1);
      stnt(s_tile4[i], dst + i);
    }
    wave_lds_handoff();
  }

  // the partial last tile, by the one wave whose sequence reaches it
  const long row0 = wt * kWave;
  if (wt == nfull && row0 < a.B) {
    const int nrows = (int)(a.B - row0);
    const int count = nrows * A;
    const int m4 = count >> 2;
    const f4* src = reinterpret_cast<const f4*>(a.x + row0 * A);
    for (int i = lane; i < m4; i += kWave) s_tile4[i] = ldnt(src + i);
    if (lane < count - (m4 << 2)) s_tile[(m4 << 2) + lane] = ldnt(a.x + row0 * A + (m4 << 2) + lane);
    wave_lds_handoff();
    if (lane < nrows) {
      const long row = row0 + lane;
      cat_row_math<KA, MAXA>(a, s_tile + lane * A, A, row, load_row_t<kVclip>(a, row),
                             row_action<ActT>(a, row), ge, acc);
    }
    wave_lds_handoff();
    f4* dst = reinterpret_cast<f4*>(a.dx + row0 * A);
    for (int i = lane; i < m4; i += kWave) stnt(s_tile4[i], dst + i);
    if (lane < count - (m4 << 2)) a.dx[row0 * A + (m4 << 2) + lane] = s_tile[(m4 << 2) + lane];
  }
  store_scalar_partials(a, acc);
  if (a.finish) loss_publish<0>(a);
}

// ---------------------------------------------------------------------------
// Categorical, any A: one wave per row (lanes stride the actions).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max_f(float x) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) x = fmaxf(x, __shfl_xor(x, off, kWave));
  return x;
}
__device__ __forceinline__ float wave_sum_f(float x) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) x += __shfl_xor(x, off, kWave);
  return x;
}

template <typename ActT>
__global__ void __launch_bounds__(kBlock) loss_cat_wave_kernel(LossArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const long wave = ((long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long nwaves = (long)gridDim.x * blockDim.x / kWave;
  const int A = a.A;
  const float ge = a.ec * a.inv_b;
  double acc[5] = {0, 0, 0, 0, 0};
  for (long row = wave; row < a.B; row += nwaves) {
    const float* z = a.x + row * A;
    float m = -INFINITY;
    for (int j = lane; j < A; j += kWave) m = fmaxf(m, z[j]);
    m = wave_max_f(m);
    float s = 0.0f, S = 0.0f;
    for (int j = lane; j < A; j += kWave) {
      const float t = z[j] - m;
      const float e = __expf(t);
      s += e;
      S += e > 0.0f ? e * t : 0.0f;
    }
    s = wave_sum_f(s);
    S = wave_sum_f(S);
    const float log_s = logf(s);
    const float inv_s = 1.0f / s;
    const float H = log_s - S * inv_s;
    const int ai = row_action<ActT>(a, row);
    const float lp = ai >= 0 ? (z[ai] - m) - log_s : __builtin_nanf("");
    // every lane evaluates the row terms; only lane 0 stores dvalue and sums
    RowOut o = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (lane == 0) o = ppo_row(a, row, load_row(a, row), lp);
    o.g_lp = __shfl(o.g_lp, 0, kWave);
    float* dz = a.dx + row * A;
    for (int j = lane; j < A; j += kWave) {
      const float t = z[j] - m;
      const float p = __expf(t) * inv_s;
      const float logp = fmaxf(t - log_s, -FLT_MAX);
      const float onehot = j == ai ? 1.0f : 0.0f;
      dz[j] = o.g_lp * (onehot - p) + ge * (p * (logp + H));
    }
    if (lane == 0) accumulate(acc, o, H);
  }
  store_scalar_partials(a, acc);
  if (a.finish) loss_publish<0>(a);
}

// ---------------------------------------------------------------------------
// Gaussian, D <= kMaxGaussDim: one thread per row; mu and actions staged
// through LDS.  torch Normal(loc, scale): log_prob = -(x-loc)^2/(2*scale^2)
// - log(scale) - log(sqrt(2*pi)); entropy = 0.5 + 0.5*log(2*pi) + log(scale)
// (constant over rows; the finaliser forms it).  The divisions by 2*var and
// var are multiplications by per-dim reciprocals computed once per block
// (<= 1 ulp from torch's quotient).
// ---------------------------------------------------------------------------
template <bool kVec>
__global__ void __launch_bounds__(kBlock) loss_gauss_kernel(LossArgs a, long ntiles) {
  extern __shared__ float s_lds[];
  __shared__ float s_inv2var[kMaxGaussDim], s_invvar[kMaxGaussDim], s_logscale[kMaxGaussDim];
  __shared__ double s_col[kBlock];
  const int D = a.A;
  const int DS = D | 1;
  const float invD = 1.0f / (float)D;
  float* s_mu = s_lds;
  float* s_act = s_lds + kBlock * DS;
  const float kLogSqrt2Pi = 0.91893853320467274178f;   // log(sqrt(2*pi))
  const int tid = threadIdx.x;
  if (tid < D) {
    const float scale = expf(a.log_std[tid]);
    const float var = scale * scale;
    s_inv2var[tid] = 1.0f / (2.0f * var);
    s_invvar[tid] = 1.0f / var;
    s_logscale[tid] = logf(scale);
  }
  const int groups = kBlock / D;
  double col_acc = 0.0;  // thread t < D: this block's dlog_std[t] over its tiles
  double acc[5] = {0, 0, 0, 0, 0};

  for (long tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const long row0 = tile * kBlock;
    const int nrows = (int)std::min<long>(kBlock, a.B - row0);
    const long row = row0 + tid;
    RowIn in = {0, 0, 0, 0, 0};
    if (tid < nrows) in = load_row(a, row);
    stage_in<kVec>(a.x + row0 * D, nrows * D, D, invD, DS, s_mu);
    stage_in<kVec>(reinterpret_cast<const float*>(a.actions) + row0 * D, nrows * D, D, invD, DS,
                   s_act);
    __syncthreads();
    if (tid < nrows) {
      float* mu = s_mu + tid * DS;
      float* act = s_act + tid * DS;
      float lp = 0.0f;
      for (int d = 0; d < D; ++d) {
        const float diff = act[d] - mu[d];
        lp += ((-(diff * diff)) * s_inv2var[d] - s_logscale[d]) - kLogSqrt2Pi;
      }
      const RowOut o = ppo_row(a, row, in, lp);
      for (int d = 0; d < D; ++d) {
        const float diff = act[d] - mu[d];
        const float z2 = (diff * diff) * s_invvar[d];
        mu[d] = o.g_lp * (diff * s_invvar[d]);  // dmu
        act[d] = o.g_lp * (z2 - 1.0f);       // this row's dlog_std term
      }
      accumulate(acc, o, 0.0f);
    } else {
      float* act = s_act + tid * DS;
      for (int d = 0; d < D; ++d) act[d] = 0.0f;
    }
    __syncthreads();
    stage_out<kVec>(a.dx + row0 * D, nrows * D, D, invD, DS, s_mu);
    // column sums of the dlog_std terms: `groups` threads per column, then
    // one thread per column, fixed order, fp64
    double sum = 0.0;
    if (tid < groups * D) {
      const int d = tid % D;
      const int g = tid / D;
      for (int r = g; r < kBlock; r += groups) sum += (double)s_act[r * DS + d];
    }
    s_col[tid] = sum;
    __syncthreads();
    if (tid < D)
      for (int g = 0; g < groups; ++g) col_acc += s_col[g * D + tid];
    __syncthreads();
  }
  if (tid < D) store_partial(a, kLossSums + tid, col_acc);
  store_scalar_partials(a, acc);
  loss_publish<kMaxGaussDim>(a);
}

// ---------------------------------------------------------------------------
// Gaussian, register-resident form for 16-byte-aligned mu/actions/dmu (any
// D <= MAXD; KD > 0 fixes D at compile time).  mu and action tiles are staged
// in LDS in their global layout (ds_write_b128, no index arithmetic), each
// thread reads its row of both into registers, and this block's dlog_std
// column sums accumulate in per-thread fp64 registers across all its tiles
// (one block reduction per dim at the end) instead of an LDS column pass per
// tile.  Per element: diff, diff^2, an FMA into log_prob, dmu and the
// dlog_std term.
// ---------------------------------------------------------------------------
template <int PF>
struct GaussPrefetch {
  f4 mu[PF], act[PF];
  float mu_tail, act_tail;
  RowIn in;
  int nrows;
};

template <int PF>
__device__ __forceinline__ void gauss_prefetch(const LossArgs& a, long tile, int D,
                                               GaussPrefetch<PF>& p) {
  const int tid = threadIdx.x;
  const long row0 = tile * kBlock;
  p.nrows = (int)std::min<long>(kBlock, a.B - row0);
  const int count = p.nrows * D;
  const int n4 = count >> 2;
  const f4* m4 = reinterpret_cast<const f4*>(a.x + row0 * D);
  const f4* a4 = reinterpret_cast<const f4*>(reinterpret_cast<const float*>(a.actions) + row0 * D);
#pragma unroll
  for (int k = 0; k < PF; ++k) {
    const int i = k * kBlock + tid;
    if (i < n4) {
      p.mu[k] = ldnt(m4 + i);
      p.act[k] = ldnt(a4 + i);
    }
  }
  if (tid < count - (n4 << 2)) {
    p.mu_tail = ldnt(a.x + row0 * D + (n4 << 2) + tid);
    p.act_tail = ldnt(reinterpret_cast<const float*>(a.actions) + row0 * D + (n4 << 2) + tid);
  }
  if (tid < p.nrows) p.in = load_row(a, row0 + tid);
}

template <int KD, int MAXD>
__global__ void __launch_bounds__(kBlock) loss_gauss_dense_kernel(LossArgs a, long ntiles) {
  constexpr int PF = (MAXD + 3) / 4;
  extern __shared__ float s_lds[];
  __shared__ float s_inv2var[kMaxGaussDim], s_invvar[kMaxGaussDim], s_logscale[kMaxGaussDim];
  const int D = KD > 0 ? KD : a.A;
  float* s_mu = s_lds;
  float* s_act = s_lds + kBlock * D;
  f4* s_mu4 = reinterpret_cast<f4*>(s_mu);
  f4* s_act4 = reinterpret_cast<f4*>(s_act);
  const float kLogSqrt2Pi = 0.91893853320467274178f;  // log(sqrt(2*pi))
  const int tid = threadIdx.x;
  if (tid < D) {
    const float scale = expf(a.log_std[tid]);
    const float var = scale * scale;
    s_inv2var[tid] = 1.0f / (2.0f * var);
    s_invvar[tid] = 1.0f / var;
    s_logscale[tid] = logf(scale);
  }
  double col[MAXD];
#pragma unroll
  for (int d = 0; d < MAXD; ++d) col[d] = 0.0;
  double acc[5] = {0, 0, 0, 0, 0};
  GaussPrefetch<PF> pf;
  long tile = blockIdx.x;
  if (tile < ntiles) gauss_prefetch<PF>(a, tile, D, pf);

  for (; tile < ntiles; tile += gridDim.x) {
    const int nrows = pf.nrows;
    const int count = nrows * D;
    const int n4 = count >> 2;
#pragma unroll
    for (int k = 0; k < PF; ++k) {
      const int i = k * kBlock + tid;
      if (i < n4) {
        s_mu4[i] = pf.mu[k];
        s_act4[i] = pf.act[k];
      }
    }
    if (tid < count - (n4 << 2)) {
      s_mu[(n4 << 2) + tid] = pf.mu_tail;
      s_act[(n4 << 2) + tid] = pf.act_tail;
    }
    const RowIn in = pf.in;
    const long row0 = tile * kBlock;
    __syncthreads();

    const long next = tile + gridDim.x;
    if (next < ntiles) gauss_prefetch<PF>(a, next, D, pf);

    if (tid < nrows) {
      float* mu = s_mu + tid * D;
      const float* act = s_act + tid * D;
      float diff[MAXD];
      float lp = 0.0f;
#pragma unroll
      for (int d = 0; d < MAXD; ++d)
        if (d < D) {
          diff[d] = act[d] - mu[d];
          lp += ((-(diff[d] * diff[d])) * s_inv2var[d] - s_logscale[d]) - kLogSqrt2Pi;
        }
      const RowOut o = ppo_row(a, row0 + tid, in, lp);
#pragma unroll
      for (int d = 0; d < MAXD; ++d)
        if (d < D) {
          const float z = diff[d] * s_invvar[d];
          mu[d] = o.g_lp * z;                                        // dmu
          col[d] += (double)(o.g_lp * (diff[d] * z - 1.0f));         // dlog_std term
        }
      accumulate(acc, o, 0.0f);
    }
    __syncthreads();
    f4* dst = reinterpret_cast<f4*>(a.dx + row0 * D);
    for (int i = tid; i < n4; i += kBlock) stnt(s_mu4[i], dst + i);
    if (tid < count - (n4 << 2)) a.dx[row0 * D + (n4 << 2) + tid] = s_mu[(n4 << 2) + tid];
    __syncthreads();
  }
  // this block's loss sums and dlog_std column sums: one block reduction
  double all[kLossSums + MAXD];
#pragma unroll
  for (int k = 0; k < kLossSums; ++k) all[k] = acc[k];
#pragma unroll
  for (int d = 0; d < MAXD; ++d) all[kLossSums + d] = col[d];
  block_sum<kLossSums + MAXD>(all);
  if (tid == 0) {
#pragma unroll
    for (int k = 0; k < kLossSums + MAXD; ++k)
      if (k < kLossSums + D) store_partial(a, k, all[k]);
  }
  loss_publish<MAXD>(a);
}

// ---------------------------------------------------------------------------
// Gaussian, wave tiles (16-byte-aligned mu/actions/dmu, D <= MAXD <= 8; KD >
// 0 fixes D at compile time): the categorical wave-tile scheme applied to the
// Gaussian policy (B = 2,097,152, D = 6: 48.8 us per call against 49.6-50.0 us for
// the 256-row dense kernel).  Each wave owns tiles of 64 consecutive rows (one
// contiguous span of 64*D floats of mu and of actions: 16*D float4 each),
// staged through its own LDS slice in their global layout, so no workgroup
// barrier is needed in the loop; the next tile's loads are issued before the
// current tile's arithmetic.  Full tiles run branch-free (clamped float4
// indices: lanes past the end repeat the last float4, same address, same
// value); the partial last tile (B mod 64 rows) is processed after the loop.
// The per-row arithmetic is the dense kernel's, operation for operation.
// ---------------------------------------------------------------------------
template <int PF>
struct GaussWavePrefetch {
  f4 mu[PF], act[PF];
  RowIn in;
};

template <int PF, bool kVclip>
__device__ __forceinline__ void gauss_wave_prefetch(const LossArgs& a, long wt, int lane, int D,
                                                    GaussWavePrefetch<PF>& p) {
  const long row0 = wt * kWave;
  const int n4 = (kWave / 4) * D;
  const f4* m4 = reinterpret_cast<const f4*>(a.x + row0 * D);
  const f4* a4 =
      reinterpret_cast<const f4*>(reinterpret_cast<const float*>(a.actions) + row0 * D);
#pragma unroll
  for (int k = 0; k < PF; ++k) {
    const int i = std::min(k * kWave + lane, n4 - 1);
    p.mu[k] = ldnt(m4 + i);
    p.act[k] = ldnt(a4 + i);
  }
  __builtin_amdgcn_sched_barrier(0);
  p.in = load_row_t<kVclip>(a, row0 + lane);
}

// One row: log-prob, the PPO row terms, dmu in place of mu, the dlog_std
// column terms and the loss sums.
template <int MAXD>
__device__ __forceinline__ void gauss_row_math(const LossArgs& a, float* mu, const float* act,
                                               int D, long row, const RowIn& in,
                                               const float* inv2var, const float* invvar,
                                               const float* logscale, double (&col)[MAXD],
                                               double (&acc)[5]) {
  const float kLogSqrt2Pi = 0.91893853320467274178f;  // log(sqrt(2*pi))
  float diff[MAXD];
  float lp = 0.0f;
#pragma unroll
  for (int d = 0; d < MAXD; ++d)
    if (d < D) {
      diff[d] = act[d] - mu[d];
      lp += ((-(diff[d] * diff[d])) * inv2var[d] - logscale[d]) - kLogSqrt2Pi;
    }
  const RowOut o = ppo_row(a, row, in, lp);
#pragma unroll
  for (int d = 0; d < MAXD; ++d)
    if (d < D) {
      const float z = diff[d] * invvar[d];
      mu[d] = o.g_lp * z;                                 // dmu
      col[d] += (double)(o.g_lp * (diff[d] * z - 1.0f));  // dlog_std term
    }
  accumulate(acc, o, 0.0f);
}

template <int KD, int MAXD, bool kVclip>
__global__ void __launch_bounds__(kBlock) loss_gauss_wtile_kernel(LossArgs a, long nfull) {
  constexpr int PF = (MAXD + 3) / 4;
  constexpr int kWavesPerBlock = kBlock / kWave;
  extern __shared__ float s_lds[];
  __shared__ float s_inv2var[kMaxGaussDim], s_invvar[kMaxGaussDim], s_logscale[kMaxGaussDim];
  const int D = KD > 0 ? KD : a.A;
  const int n4 = (kWave / 4) * D;  // float4 per full tile and array
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wid = tid / kWave;
  float* s_mu = s_lds + wid * 2 * kWave * D;  // 256*D bytes per array: 16-byte aligned
  float* s_act = s_mu + kWave * D;
  f4* s_mu4 = reinterpret_cast<f4*>(s_mu);
  f4* s_act4 = reinterpret_cast<f4*>(s_act);
  if (tid < D) {
    const float scale = expf(a.log_std[tid]);
    const float var = scale * scale;
    s_inv2var[tid] = 1.0f / (2.0f * var);
    s_invvar[tid] = 1.0f / var;
    s_logscale[tid] = logf(scale);
  }
  __syncthreads();
  double col[MAXD];
#pragma unroll
  for (int d = 0; d < MAXD; ++d) col[d] = 0.0;
  double acc[5] = {0, 0, 0, 0, 0};
  GaussWavePrefetch<PF> pf;
  // (with a.collector = c, workgroups 0 .. c-1 take no tiles: they only collect)
  const long c0 = a.collector;
  const long wstride = ((long)gridDim.x - c0) * kWavesPerBlock;
  long wt = (long)blockIdx.x < c0 ? nfull + 1 : ((long)blockIdx.x - c0) * kWavesPerBlock + wid;
  if (wt < nfull) gauss_wave_prefetch<PF, kVclip>(a, wt, lane, D, pf);

  for (; wt < nfull; wt += wstride) {
#pragma unroll
    for (int k = 0; k < PF; ++k) {
      const int i = std::min(k * kWave + lane, n4 - 1);
      s_mu4[i] = pf.mu[k];
      s_act4[i] = pf.act[k];
    }
    const RowIn in = pf.in;
    const long row0 = wt * kWave;
    wave_lds_handoff();

    const long next = wt + wstride;
    if (next < nfull) gauss_wave_prefetch<PF, kVclip>(a, next, lane, D, pf);

    gauss_row_math<MAXD>(a, s_mu + lane * D, s_act + lane * D, D, row0 + lane, in, s_inv2var,
                         s_invvar, s_logscale, col, acc);
    wave_lds_handoff();
    f4* dst = reinterpret_cast<f4*>(a.dx + row0 * D);
#pragma unroll
    for (int k = 0; k < PF; ++k) {
      const int i = std::min(k * kWave + lane, n4 - 1);
      stnt(s_mu4[i], dst + i);
    }
    wave_lds_handoff();
  }

  // the partial last tile, by the one wave whose sequence reaches it
  const long row0 = wt * kWave;
  if (wt == nfull && row0 < a.B) {
    const int nrows = (int)(a.B - row0);
    const int count = nrows * D;
    const int m4 = count >> 2;
    const float* mu_src = a.x + row0 * D;
    const float* act_src = reinterpret_cast<const float*>(a.actions) + row0 * D;
    for (int i = lane; i < m4; i += kWave) {
      s_mu4[i] = ldnt(reinterpret_cast<const f4*>(mu_src) + i);
      s_act4[i] = ldnt(reinterpret_cast<const f4*>(act_src) + i);
    }
    if (lane < count - (m4 << 2)) {
      s_mu[(m4 << 2) + lane] = ldnt(mu_src + (m4 << 2) + lane);
      s_act[(m4 << 2) + lane] = ldnt(act_src + (m4 << 2) + lane);
    }
    wave_lds_handoff();
    if (lane < nrows)
      gauss_row_math<MAXD>(a, s_mu + lane * D, s_act + lane * D, D, row0 + lane,
                           load_row_t<kVclip>(a, row0 + lane), s_inv2var, s_invvar, s_logscale,
                           col, acc);
    wave_lds_handoff();
    f4* dst = reinterpret_cast<f4*>(a.dx + row0 * D);
    for (int i = lane; i < m4; i += kWave) stnt(s_mu4[i], dst + i);
    if (lane < count - (m4 << 2)) a.dx[row0 * D + (m4 << 2) + lane] = s_mu[(m4 << 2) + lane];
  }
  // this block's loss sums and dlog_std column sums: one block reduction
  double all[kLossSums + MAXD];
#pragma unroll
  for (int k = 0; k < kLossSums; ++k) all[k] = acc[k];
#pragma unroll
  for (int d = 0; d < MAXD; ++d) all[kLossSums + d] = col[d];
  block_sum<kLossSums + MAXD>(all);
  if (tid == 0) {
#pragma unroll
    for (int k = 0; k < kLossSums + MAXD; ++k)
      if (k < kLossSums + D) store_partial(a, k, all[k]);
  }
  loss_publish<MAXD>(a);
}

#ifndef PPO_GAUSS_WTILE
#define PPO_GAUSS_WTILE 1  // build-time switch: 0 keeps the 256-row dense kernel
#endif

int fill_common(LossArgs& a, long B, const ppo_loss_params* p, const float* old_lp,
                const float* adv, const float* ret, const float* val, const float* old_val,
                float* dval, float* scalars) {
  if (!p || !old_lp || !adv || !ret || !val || !dval || !scalars) return PPO_ERR_INVALID_ARG;
  if (!(p->clip_ratio >= 0.0)) return PPO_ERR_INVALID_ARG;
  a.B = B;
  a.old_lp = old_lp;
  a.adv = adv;
  a.ret = ret;
  a.val = val;
  a.old_val = old_val;
  const RowParams rp = make_row_params(p, B);
  a.lo = rp.lo;
  a.hi = rp.hi;
  a.clip = rp.clip;
  a.use_vclip = rp.use_vclip;
  if (a.use_vclip && !old_val) return PPO_ERR_INVALID_ARG;
  a.vclip = rp.vclip;
  a.vc = rp.vc;
  a.ec = rp.ec;
  a.inv_b = rp.inv_b;
  a.dval = dval;
  a.scalars = scalars;
  return PPO_OK;
}

long row_tiles(long B) { return (B + kBlock - 1) / kBlock; }

// How the categorical loss forms its scalars: in-kernel (loss_publish:
// every workgroup tags its partials and workgroup 0 collects them) or by the
// one-block finaliser launch after the kernel.  Measured on MI355X (A = 18):
//  - collected by a working workgroup, in-kernel beats the launch at B =
//    1,048,576 (40.9 against 42.4 us per call) but not inside the PPO step
//    at B = 8,388,608 (260.6 against 257.5 us): the collector's polls are
//    queued behind its own wave's outstanding gradient stores (one in-order
//    counter per wave for loads and stores);
//  - collected by a workgroup that takes no tiles (wave-tile kernels, the
//    other workgroups share its tiles), the polls return at once: B =
//    8,388,608 in the step 258.2-258.4 against 261.2-262.4 us, step 291.9-292.4
//    against 295.3-296.0 us; B = 1,048,576 40.4-40.5 against 40.7-41.0 us.
// So the wave-tile kernels finish in-kernel with a dedicated collector at
// every batch size, the other forms in-kernel up to kCatFinishRows rows.
// PPO_AMD_CAT_FINISH=0 selects the finaliser launch everywhere (no
// in-kernel wait: for callers that share the GPU).
constexpr long kCatFinishRows = 1L << 22;

bool cat_finish_in_kernel() {
  const char* env = getenv("PPO_AMD_CAT_FINISH");
  return !(env && env[0] == '0');
}

long cat_blocks(long B, int A) {
  if (A <= kMaxCatRowWidth) return std::min(row_tiles(B), kLossGridCap);
  return std::max(1L, std::min((B + 3) / 4, kWaveRowBlocks));
}

long gauss_blocks(long B) { return std::min(row_tiles(B), kLossGridCap); }

dim3 grid_of(long blocks) { return dim3((unsigned)blocks); }

}  // namespace
}  // namespace ppo

extern "C" size_t ppo_loss_cat_workspace_bytes(int64_t B, int32_t A) {
  using namespace ppo;
  if (B <= 0 || A <= 0) return kHeaderBytes;
  return kHeaderBytes + align_up((size_t)cat_blocks(B, A) * kScalarSlots * sizeof(double), 256);
}

namespace ppo {
namespace {

// Argument checks of ppo_loss_cat_f32 that come before the workspace check.
int loss_cat_check(const float* logits, int64_t B, int32_t A, const void* actions,
                   const float* dlogits) {
  if (B <= 0 || A <= 0) return PPO_ERR_INVALID_ARG;
  if (!logits || !actions || !dlogits) return PPO_ERR_INVALID_ARG;
  if ((long)B * A > (1L << 50)) return PPO_ERR_TOO_LARGE;
  return PPO_OK;
}

// ppo_loss_cat_f32 after its checks; `workspace` holds at least
// ppo_loss_cat_workspace_bytes(B, A) bytes of device memory.
int loss_cat_launch(const float* logits, int64_t B, int32_t A, const void* actions,
                    int actions_are_int64, const float* old_log_probs, const float* advantages,
                    const float* returns, const float* values, const float* old_values,
                    const ppo_loss_params* params, float* dlogits, float* dvalues,
                    float* scalars_out, void* workspace, void* stream_ptr) {
  LossArgs a = {};
  int st = fill_common(a, B, params, old_log_probs, advantages, returns, values, old_values,
                       dvalues, scalars_out);
  if (st) return st;
  a.x = logits;
  a.A = A;
  a.actions = actions;
  a.dx = dlogits;
  a.partial = reinterpret_cast<double*>(static_cast<char*>(workspace) + kHeaderBytes);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  long blocks = cat_blocks(B, A);
  const long tiles = row_tiles(B);
  if (A <= kMaxCatRowWidth) {
    const bool vec = aligned(logits, 16) && aligned(dlogits, 16);
    size_t lds = (size_t)kBlock * (A | 1) * sizeof(float);
    const void* kern;
    const bool dense = vec && (A % 4) != 0 && A <= 20;
    const bool vclip = a.use_vclip != 0;
#define PPO_DENSE(KA, M)                                                                 \
  (actions_are_int64                                                                     \
       ? (vclip ? (const void*)loss_cat_wtile_kernel<int64_t, KA, M, true>               \
                : (const void*)loss_cat_wtile_kernel<int64_t, KA, M, false>)             \
       : (vclip ? (const void*)loss_cat_wtile_kernel<int32_t, KA, M, true>               \
                : (const void*)loss_cat_wtile_kernel<int32_t, KA, M, false>))
    if (dense && A == 2)
      kern = PPO_DENSE(2, 2);
    else if (dense && A == 3)
      kern = PPO_DENSE(3, 3);
    else if (dense && A == 5)
      kern = PPO_DENSE(5, 5);
    else if (dense && A == 6)
      kern = PPO_DENSE(6, 6);
    else if (dense && A == 7)
      kern = PPO_DENSE(7, 7);
    else if (dense && A == 9)
      kern = PPO_DENSE(9, 9);
    else if (dense && A == 18)
      kern = PPO_DENSE(18, 18);
    else if (dense && A <= 4)
      kern = PPO_DENSE(0, 4);
    else if (dense && A <= 8)
      kern = PPO_DENSE(0, 8);
    else if (dense && A <= 12)
      kern = PPO_DENSE(0, 12);
    else if (dense)
      kern = PPO_DENSE(0, 20);
#undef PPO_DENSE
    else if (vec && (A + 3) / 4 <= 2)
      kern = actions_are_int64 ? (const void*)loss_cat_pipe_kernel<int64_t, 2>
                               : (const void*)loss_cat_pipe_kernel<int32_t, 2>;
    else if (vec && (A + 3) / 4 <= 5)
      kern = actions_are_int64 ? (const void*)loss_cat_pipe_kernel<int64_t, 5>
                               : (const void*)loss_cat_pipe_kernel<int32_t, 5>;
    else if (vec)
      kern = actions_are_int64 ? (const void*)loss_cat_kernel<int64_t, true>
                               : (const void*)loss_cat_kernel<int32_t, true>;
    else
      kern = actions_are_int64 ? (const void*)loss_cat_kernel<int64_t, false>
                               : (const void*)loss_cat_kernel<int32_t, false>;
    if (dense) lds = (size_t)kBlock * A * sizeof(float);
    // one wave of resident workgroups looping over the tiles
    const long resident = resident_blocks(kern, kBlock, lds, 0);
    blocks = std::min(blocks, resident > 0 ? resident : blocks);
    // in-kernel finish (cat_finish_in_kernel), for a grid resident at once
    if (resident > 0 && cat_finish_in_kernel() && (dense ? blocks > 1 : B <= kCatFinishRows)) {
      a.collector = dense ? 1 : 0;
      int wst = wait_ctl(a.wc);
      if (wst) return wst;
      a.finish = 1;
      a.epoch = &static_cast<WsHeader*>(workspace)->epoch;
      a.tag_slot = kScalarSlots - 1;
    }
    const long wfull = B / kWave;  // full wave tiles
    void* args[] = {&a, const_cast<long*>(dense ? &wfull : &tiles)};
    st = hip_status(hipLaunchKernel(kern, grid_of(blocks), dim3(kBlock), args, lds, stream));
    if (st) return st;
  } else {
    if (actions_are_int64)
      hipLaunchKernelGGL(loss_cat_wave_kernel<int64_t>, dim3((unsigned)blocks), dim3(kBlock), 0,
                         stream, a);
    else
      hipLaunchKernelGGL(loss_cat_wave_kernel<int32_t>, dim3((unsigned)blocks), dim3(kBlock), 0,
                         stream, a);
  }
  if ((st = last_launch_status())) return st;
  if (a.finish) return PPO_OK;
  hipLaunchKernelGGL(loss_finalize_kernel, dim3(1), dim3(kFinalBlock), 0, stream, a, blocks);
  return last_launch_status();
}

}  // namespace

// Scratch of the allocation-free entry point: the per-workgroup partial sums
// of the largest grid either categorical kernel family launches, behind the
// workspace header.  One copy per device, zero-initialised at load and held
// until the process ends; every call on a device reuses it.
constexpr size_t kLossScratchBytes =
    kHeaderBytes + (size_t)(kWaveRowBlocks > kLossGridCap ? kWaveRowBlocks : kLossGridCap) *
                       kScalarSlots * sizeof(double);
__device__ __align__(256) unsigned char scratch[kLossScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// Device address of `scratch` on the current device, looked up once per
// device with that device current.  In host code the name `scratch` is only
// a host-side handle: kernels must be given this address.
int scratch_address(void** out) {
  int dev = 0;
  int st = hip_status(hipGetDevice(&dev));
  if (st) return st;
  if (dev < 0 || dev >= kMaxDevices) return PPO_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if ((st = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))))) return st;
    if (!p) return PPO_ERR_HIP_BASE + (int)hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PPO_OK;
}

}  // namespace

int scratch_clear(hipStream_t stream) {
  void* p = nullptr;
  int st = scratch_address(&p);
  if (st) return st;
  return hip_status(hipMemsetAsync(p, 0, kLossScratchBytes, stream));
}

}  // namespace ppo

extern "C" int ppo_loss_cat_f32(const float* logits, int64_t B, int32_t A, const void* actions,
                                int actions_are_int64, const float* old_log_probs,
                                const float* advantages, const float* returns,
                                const float* values, const float* old_values,
                                const ppo_loss_params* params, float* dlogits, float* dvalues,
                                float* scalars_out, void* workspace, size_t workspace_bytes,
                                void* stream_ptr) {
  using namespace ppo;
  int st = loss_cat_check(logits, B, A, actions, dlogits);
  if (st) return st;
  if (!workspace || workspace_bytes < ppo_loss_cat_workspace_bytes(B, A)) return PPO_ERR_WORKSPACE;
  return loss_cat_launch(logits, B, A, actions, actions_are_int64, old_log_probs, advantages,
                         returns, values, old_values, params, dlogits, dvalues, scalars_out,
                         workspace, stream_ptr);
}

extern "C" int ppo_loss_cat_f32_noalloc(const float* logits, int64_t B, int32_t A,
                                        const void* actions, int actions_are_int64,
                                        const float* old_log_probs, const float* advantages,
                                        const float* returns, const float* values,
                                        const float* old_values, const ppo_loss_params* params,
                                        float* dlogits, float* dvalues, float* scalars_out,
                                        void* stream_ptr) {
  using namespace ppo;
  int st = loss_cat_check(logits, B, A, actions, dlogits);
  if (st) return st;
  if (ppo_loss_cat_workspace_bytes(B, A) > kLossScratchBytes) return PPO_ERR_TOO_LARGE;
  void* ws = nullptr;
  if ((st = scratch_address(&ws))) return st;
  return loss_cat_launch(logits, B, A, actions, actions_are_int64, old_log_probs, advantages,
                         returns, values, old_values, params, dlogits, dvalues, scalars_out, ws,
                         stream_ptr);
}

extern "C" size_t ppo_loss_gauss_workspace_bytes(int64_t B, int32_t D) {
  using namespace ppo;
  if (B <= 0 || D <= 0) return kHeaderBytes;
  return kHeaderBytes + align_up((size_t)gauss_blocks(B) * kGaussSlots * sizeof(double), 256);
}

extern "C" int ppo_loss_gauss_f32(const float* mu, const float* log_std, int64_t B, int32_t D,
                                  const float* actions, const float* old_log_probs,
                                  const float* advantages, const float* returns,
                                  const float* values, const float* old_values,
                                  const ppo_loss_params* params, float* dmu, float* dlog_std,
                                  float* dvalues, float* scalars_out, void* workspace,
                                  size_t workspace_bytes, void* stream_ptr) {
  using namespace ppo;
  if (B <= 0 || D <= 0) return PPO_ERR_INVALID_ARG;
  if (D > kMaxGaussDim) return PPO_ERR_TOO_LARGE;
  if (!mu || !log_std || !actions || !dmu || !dlog_std) return PPO_ERR_INVALID_ARG;
  if ((long)B * D > (1L << 50)) return PPO_ERR_TOO_LARGE;
  if (!workspace || workspace_bytes < ppo_loss_gauss_workspace_bytes(B, D))
    return PPO_ERR_WORKSPACE;
  LossArgs a = {};
  int st = fill_common(a, B, params, old_log_probs, advantages, returns, values, old_values,
                       dvalues, scalars_out);
  if (st) return st;
  a.x = mu;
  a.log_std = log_std;
  a.A = D;
  a.actions = actions;
  a.dx = dmu;
  a.dlog_std = dlog_std;
  a.partial = reinterpret_cast<double*>(static_cast<char*>(workspace) + kHeaderBytes);
  a.epoch = &static_cast<WsHeader*>(workspace)->epoch;
  a.tag_slot = kGaussSlots - 1;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);
  long blocks = gauss_blocks(B);
  const long tiles = row_tiles(B);
  const size_t lds = (size_t)2 * kBlock * (D | 1) * sizeof(float);
  const bool vec = aligned(mu, 16) && aligned(actions, 16) && aligned(dmu, 16);
  const void* kern;
  size_t lds_used = lds;
  const long wfull = B / kWave;  // full wave tiles (wave-tile kernels)
  bool wave_tiles = false;
  if (vec && PPO_GAUSS_WTILE && D <= 8) {
    // wave tiles: each wave's 64 x D slices of mu and actions, no padding
    // (wider D stays on the dense kernel: its fp64 column sums alone would
    // need 32-48 VGPRs per lane here)
    lds_used = (size_t)2 * kBlock * D * sizeof(float);
    wave_tiles = true;
    const bool vclip = a.use_vclip != 0;
#define PPO_GW(KD, MAXD)                                                   \
  (vclip ? (const void*)loss_gauss_wtile_kernel<KD, MAXD, true>             \
         : (const void*)loss_gauss_wtile_kernel<KD, MAXD, false>)
    if (D == 6)
      kern = PPO_GW(6, 6);
    else if (D <= 4)
      kern = PPO_GW(0, 4);
    else
      kern = PPO_GW(0, 8);
#undef PPO_GW
  } else if (vec) {
    // dense layout: two 256 x D tiles, no padding
    lds_used = (size_t)2 * kBlock * D * sizeof(float);
    if (D == 6)
      kern = (const void*)loss_gauss_dense_kernel<6, 6>;
    else if (D <= 4)
      kern = (const void*)loss_gauss_dense_kernel<0, 4>;
    else if (D <= 8)
      kern = (const void*)loss_gauss_dense_kernel<0, 8>;
    else if (D <= 16)
      kern = (const void*)loss_gauss_dense_kernel<0, 16>;
    else
      kern = (const void*)loss_gauss_dense_kernel<0, 24>;
  } else {
    kern = (const void*)loss_gauss_kernel<false>;
  }
  // The in-kernel finish needs the whole grid resident at once: the grid is
  // capped at the occupancy query's answer.  When the runtime cannot answer
  // (or PPO_AMD_GAUSS_FINISH=0 is set, for callers that share the GPU), the
  // workgroups only publish and a one-workgroup launch collects after them.
  const long resident = resident_blocks(kern, kBlock, lds_used, 0);
  const char* env = getenv("PPO_AMD_GAUSS_FINISH");
  a.finish = resident > 0 && !(env && env[0] == '0');
  if (a.finish) {
    blocks = std::min(blocks, resident);
    if ((st = wait_ctl(a.wc))) return st;
    // Above 2^22 rows the D + 1 collecting workgroups take no tiles (as the
    // categorical wave-tile kernels' workgroup 0): their polls are then not
    // queued behind their own gradient stores.  Measured on MI355X (D = 6,
    // one call after a cache-evicting read): B = 8,388,608 151.9-152.5 us
    // against 155.0-156.5; B = 2,097,152 45.0-45.1 against 44.7-45.0, so
    // smaller batches keep working collectors.
    if (wave_tiles && blocks > D + 1 && B > (1L << 22)) a.collector = D + 1;
  }
  void* args[] = {&a, const_cast<long*>(wave_tiles ? &wfull : &tiles)};
  if ((st = hip_status(
           hipLaunchKernel(kern, grid_of(blocks), dim3(kBlock), args, lds_used, stream))))
    return st;
  if (a.finish) return PPO_OK;
  if ((st = wait_ctl(a.wc))) return st;
  hipLaunchKernelGGL(loss_gauss_finish_kernel<kMaxGaussDim>, dim3((unsigned)(D + 1)),
                     dim3(kBlock), 0, stream, a, blocks);
  return last_launch_status();
}
