/*
 * ppo_amd.h — C ABI of the MI355X (gfx950) PPO-update library `libppo_amd.so`.
 *
 * The reference (mrhooray/zero-to-hero, rl/deep) has no FFI: its PPO update is
 * the Python method surface of `PPOAgent` (rl/deep/agents/ppo.py:113-193).  Each
 * entry point below replaces one piece of that surface; the citation above each
 * declaration names the reference lines whose arithmetic it performs.  The
 * Python host package (`ppo_amd`) binds these symbols with ctypes and keeps the
 * reference's method names and signatures on top of them.
 *
 * Conventions shared by every entry point
 *   - All array pointers are DEVICE pointers owned by the caller.  Nothing here
 *     allocates or frees memory.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Every call only
 *     enqueues work on that stream: no host synchronisation, no device-wide
 *     synchronisation.
 *   - `workspace` is caller-owned device scratch of at least the size returned
 *     by the matching *_workspace_bytes() query; its contents on entry do not
 *     matter.  Two calls that share one workspace must be ordered (same
 *     stream, or synchronised).
 *   - Layouts are dense and row-major.  Rollout arrays are "[T,N]
 *     env-contiguous": element (t, n) lives at index t*N + n.
 *   - Return value: PPO_OK (0) or one of the PPO_ERR_* codes; codes
 *     >= PPO_ERR_HIP_BASE are PPO_ERR_HIP_BASE + hipError_t of a failed launch.
 *     ppo_amd_strerror() renders any of them.
 */
#ifndef PPO_AMD_H
#define PPO_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The library is built with hidden symbol visibility; only what this header
   declares is exported. */
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

#define PPO_OK 0
#define PPO_ERR_INVALID_ARG 1     /* null pointer, negative size, bad coefficient */
#define PPO_ERR_WORKSPACE 2       /* workspace missing or smaller than required */
#define PPO_ERR_TOO_LARGE 3       /* size beyond what the kernels index (2^31 rows) */
#define PPO_ERR_UNSUPPORTED 4     /* shape or option the kernels do not implement   */
#define PPO_ERR_WAIT_TIMEOUT 5    /* a bounded in-kernel wait gave up (ppo_wait_status) */
#define PPO_ERR_HIP_BASE 1000     /* + hipError_t */

/* Library version, as MAJOR*10000 + MINOR*100 + PATCH. */
int ppo_amd_version(void);

/* Human-readable text for a return code (static storage). */
const char* ppo_amd_strerror(int code);

/*
 * Status of the bounded in-kernel waits (no counterpart in the reference: its
 * update runs on the CPU in one thread).  Four launches hold workgroups that
 * wait for one another inside the launch: the resident GAE pass
 * (ppo_gae_f32 / ppo_gae_norm_f32, PPO_GAE_ROUTE_RESIDENT), the Gaussian loss
 * with its in-kernel finish (ppo_loss_gauss_f32), the categorical loss, which
 * also finishes in-kernel (ppo_loss_cat_f32 and its _noalloc form: every batch
 * on the wave-tile kernels, whose workgroup 0 only collects, batches of at
 * most 2^22 rows on the other forms), and the fused gradient reduction + clip
 * + Adam of ppo_mlp_cat_step_f32.  Each is launched only when
 * the occupancy query says its whole grid fits on the device at once; that
 * query assumes the device's compute units are free.  When another process
 * or stream keeps part of the grid from running, a wait gives up after its
 * poll limit instead of hanging; the workgroup then writes NaN over its GAE
 * outputs or loss scalars, or leaves its share of the parameters, moments,
 * gradients and step counter unwritten, and raises a status word kept per
 * device by the library.
 *
 * ppo_wait_status enqueues a read of that word on `stream`, synchronises the
 * stream, clears the word and returns PPO_ERR_WAIT_TIMEOUT if any wait on the
 * current device gave up since the previous call (on any stream), PPO_OK
 * otherwise.  It is a host synchronisation point, for callers to place where
 * they already synchronise (the Python layer checks once per update).
 * After a give-up, a workgroup that was late may have left arrival tags and
 * counters that a later call on the same workspace would take for its own:
 * when it returns PPO_ERR_WAIT_TIMEOUT the library has zeroed the scratch of
 * ppo_loss_cat_f32_noalloc, and the caller must zero (or discard) every
 * workspace used since the previous PPO_OK before passing it again (the
 * Python layer zeroes its pooled workspaces).  A zeroed workspace is always
 * valid.
 * PPO_AMD_GAE_RESIDENT=0, PPO_AMD_GAUSS_FINISH=0, PPO_AMD_CAT_FINISH=0 and
 * PPO_AMD_MLP_FUSED_ADAM=0 select launches without in-kernel waits, for
 * callers that share the GPU.
 */
int ppo_wait_status(void* stream);

/*
 * The same take of the status word without a host synchronisation: enqueues
 * on `stream` the read-and-clear of the word and a copy of its value (0 = no
 * give-up) to *host_word, which must be pinned host memory (hipHostMalloc,
 * torch pin_memory) and is valid once the stream has passed this call (an
 * event).  For loops that check the previous iteration's status while the
 * next one runs; on a non-zero value the caller must treat every output since
 * its previous clean check as invalid, and zero its workspaces and (ppo_wait_reset)
 * the library's scratch as above.
 */
int ppo_wait_status_async(uint32_t* host_word, void* stream);

/* Zeroes the library's scratch on the current device (ordered on `stream`,
   then synchronised): what ppo_wait_status does on a give-up, for callers
   that learn of it through ppo_wait_status_async. */
int ppo_wait_reset(void* stream);

/*
 * Poll limit of every bounded wait launched after this call (process-wide;
 * tests and diagnostics).  0 makes every wait give up at once, so that the
 * failure path can be exercised with every kernel still exiting normally; a
 * negative value restores the default (2^22 polls).
 */
int ppo_set_wait_limit(int64_t polls);

/* ------------------------------------------------------------------------ */
/* GAE — generalized advantage estimation over a [T,N] rollout.             */
/* ------------------------------------------------------------------------ */

/* Scratch needed by ppo_gae_f32 / ppo_gae_norm_f32 for a T x N rollout. */
size_t ppo_gae_workspace_bytes(int64_t T, int64_t N);

/*
 * Replaces PPOAgent._advantages (rl/deep/agents/ppo.py:173-193) together with
 * `returns = advantages + old_values` (ppo.py:124), generalised from one
 * episode to N independent environments with a bootstrap value.
 *
 * For each env n, walking t from T-1 down to 0 (Python float64 semantics of
 * ppo.py:177-190, evaluated in fp64 in the same operation order):
 *     mask   = 1 - dones[t,n]                      (dones: 0/1 bytes)
 *     next_v = t+1 < T ? values[t+1,n] : last_value[n]
 *     delta  = (rewards[t,n] + (gamma*next_v)*mask) - values[t,n]
 *     adv    = delta + ((gamma*lam)*mask)*adv      (adv = 0 after step T-1)
 *     adv_out[t,n] = (float)adv
 *     ret_out[t,n] = adv_out[t,n] + values[t,n]    (fp32 add, as ppo.py:124)
 * last_value may be NULL, meaning zeros: that is the reference's own
 * end-of-episode rule (ppo.py:175-176, `next_value = 0.0`).
 * values may be NULL, meaning zeros: with lam = 1 the advantages are then the
 * discounted returns value = reward + gamma*value of REINFORCE
 * (rl/deep/agents/reinforce.py:57-63), per env, reset at dones.
 * A non-zero byte in dones counts as done.  ret_out may be NULL.
 */
int ppo_gae_f32(const float* rewards, const float* values, const uint8_t* dones,
                const float* last_value, int64_t T, int64_t N, double gamma,
                double lam, float* adv_out, float* ret_out, void* workspace,
                size_t workspace_bytes, void* stream);

/*
 * ppo_gae_f32 followed by advantage normalisation over all T*N advantages
 * (ppo.py:126-127):  if T*N > 1,
 *     adv_norm_out = (adv - mean(adv)) / (std(adv) + eps)     [std unbiased]
 * else adv_norm_out = adv.  mean and std are accumulated in fp64 during the
 * GAE pass and rounded to fp32; the final expression is evaluated in fp32.
 * adv_norm_out may alias adv_out (normalisation in place, as ppo.py:127 keeps
 * only the normalised advantages; the unnormalised ones are then not stored at
 * all on the single-launch route, which saves a third of the writes).
 * stats_out (may be NULL) receives {mean, std} as two floats.
 */
int ppo_gae_norm_f32(const float* rewards, const float* values,
                     const uint8_t* dones, const float* last_value, int64_t T,
                     int64_t N, double gamma, double lam, double eps,
                     float* adv_out, float* ret_out, float* adv_norm_out,
                     float* stats_out, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Which kernels ppo_gae_f32 (normalize = 0) or ppo_gae_norm_f32 (1) run for
 * a T x N rollout with 16-byte-aligned buffers on the current device, as one
 * of the PPO_GAE_ROUTE_* values (diagnostics and tests; no counterpart in the
 * reference).  has_values = 0 means values == NULL.  Misaligned buffers take
 * the scalar tile passes whatever this returns.  The environment variable
 * PPO_AMD_GAE_RESIDENT=0 turns the resident pass off.
 */
#define PPO_GAE_ROUTE_NONE 0      /* empty or oversized rollout                */
#define PPO_GAE_ROUTE_RESIDENT 1  /* one launch, whole rollout in registers    */
#define PPO_GAE_ROUTE_STRIP 2     /* strip walk (+ normalise pass)             */
#define PPO_GAE_ROUTE_SPAN 3      /* span passes + carry scan (+ normalise)    */
#define PPO_GAE_ROUTE_TILES 4     /* tile passes + carry scan                  */
int ppo_gae_route(int64_t T, int64_t N, int normalize, int has_values);

/* ------------------------------------------------------------------------ */
/* Advantage normalisation on its own.                                      */
/* ------------------------------------------------------------------------ */

size_t ppo_adv_norm_workspace_bytes(int64_t n);

/*
 * Replaces ppo.py:126-127:
 *     if n > 1: out = (adv - adv.mean()) / (adv.std() + eps)  (unbiased std)
 *     else:     out = adv
 * out may alias adv.  stats_out (may be NULL) receives {mean, std}.
 */
int ppo_adv_norm_f32(const float* adv, int64_t n, double eps, float* out,
                     float* stats_out, void* workspace, size_t workspace_bytes,
                     void* stream);

/* ------------------------------------------------------------------------ */
/* Fused PPO loss, forward and backward in one pass.                        */
/* ------------------------------------------------------------------------ */

typedef struct ppo_loss_params {
  /* Doubles, like the Python floats of PPOConfig; the kernels round them to
     fp32 where torch's scalar-tensor arithmetic does. */
  double clip_ratio;    /* PPOConfig.clip_ratio (ppo.py:18), epsilon of the clip */
  double vf_clip;       /* value clipping range; <= 0 or +inf disables it      */
  double value_coef;    /* PPOConfig.value_coef (ppo.py:20)                     */
  double entropy_coef;  /* PPOConfig.entropy_coef (ppo.py:21)                   */
} ppo_loss_params;

/* Index of each reported scalar inside scalars_out[PPO_NUM_SCALARS]. */
#define PPO_SCALAR_LOSS 0        /* total loss (ppo.py:163-167)               */
#define PPO_SCALAR_POLICY 1      /* mean clipped-surrogate loss               */
#define PPO_SCALAR_VALUE 2       /* value loss (mse, or clipped mse)          */
#define PPO_SCALAR_ENTROPY 3     /* mean entropy                              */
#define PPO_SCALAR_APPROX_KL 4   /* mean(old_log_prob - log_prob)             */
#define PPO_SCALAR_CLIPFRAC 5    /* fraction of rows with |ratio-1| > clip     */
#define PPO_NUM_SCALARS 6

size_t ppo_loss_cat_workspace_bytes(int64_t B, int32_t A);

/*
 * Replaces the loss part of PPOAgent._update_batch (rl/deep/agents/ppo.py:150-167)
 * and its backward (ppo.py:169) down to the policy logits and the value head:
 *   dist     = Categorical(logits)          (logits [B,A])
 *   lp       = dist.log_prob(actions)       (actions [B], int32 or int64)
 *   ratio    = exp(lp - old_log_probs)
 *   policy   = -minimum(ratio*adv, clamp(ratio, 1-clip, 1+clip)*adv)
 *   value    = mse_loss(values, returns)              when vf_clip disabled
 *            = mean(maximum((v-R)^2, (v_old + clamp(v-v_old,-c,c) - R)^2))
 *   loss     = mean(policy) + value_coef*value - entropy_coef*mean(entropy)
 * Writes dloss/dlogits [B,A] and dloss/dvalues [B] (torch autograd
 * semantics, including the 1/2-1/2 split of minimum/maximum ties and the
 * inclusive clamp bounds) and scalars_out[PPO_NUM_SCALARS].
 * old_values may be NULL when vf_clip is disabled.  An action outside [0,A)
 * makes that row's log-prob NaN (the host layer validates, as torch does).
 */
int ppo_loss_cat_f32(const float* logits, int64_t B, int32_t A,
                     const void* actions, int actions_are_int64,
                     const float* old_log_probs, const float* advantages,
                     const float* returns, const float* values,
                     const float* old_values, const ppo_loss_params* params,
                     float* dlogits, float* dvalues, float* scalars_out,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * ppo_loss_cat_f32 without a workspace argument and without any allocation:
 * no counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The per-workgroup partial sums live in a library-owned
 * device array of 262,400 bytes (one copy per GPU, held until the process
 * ends), enough for every B and A ppo_loss_cat_f32 accepts; a size needing
 * more returns PPO_ERR_TOO_LARGE.  All calls on one GPU share that array, so
 * calls that overlap on one GPU (different streams, no ordering between
 * them) race and give wrong scalars; calls ordered on one stream are safe.
 * Results equal ppo_loss_cat_f32's bit for bit.
 */
int ppo_loss_cat_f32_noalloc(const float* logits, int64_t B, int32_t A,
                             const void* actions, int actions_are_int64,
                             const float* old_log_probs, const float* advantages,
                             const float* returns, const float* values,
                             const float* old_values, const ppo_loss_params* params,
                             float* dlogits, float* dvalues, float* scalars_out,
                             void* stream);

size_t ppo_loss_gauss_workspace_bytes(int64_t B, int32_t D);

/*
 * Gaussian-policy counterpart (no reference code: the reference policy is
 * categorical only, ppo.py:150).  dist = Normal(mu, exp(log_std)) with a
 * state-independent log_std[D]; log-prob and entropy are summed over the D
 * action dims (torch Normal.log_prob / Normal.entropy); the rest of the loss
 * is ppo_loss_cat_f32's.  Writes dmu [B,D], dlog_std [D] (a reduction over B),
 * dvalues [B] and scalars_out[PPO_NUM_SCALARS].  D <= 24 (PPO_ERR_TOO_LARGE
 * otherwise).
 */
int ppo_loss_gauss_f32(const float* mu, const float* log_std, int64_t B,
                       int32_t D, const float* actions,
                       const float* old_log_probs, const float* advantages,
                       const float* returns, const float* values,
                       const float* old_values, const ppo_loss_params* params,
                       float* dmu, float* dlog_std, float* dvalues,
                       float* scalars_out, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Update loop around the fused loss.                                       */
/* ------------------------------------------------------------------------ */

#define PPO_GATHER_MAX_ARRAYS 8

/*
 * Replaces the minibatch gather of PPOAgent._update (rl/deep/agents/ppo.py:
 * 132-139: observations[batch_indices], actions[batch_indices], ...): for each
 * of `narrays` (<= PPO_GATHER_MAX_ARRAYS) row-major arrays of n_src rows,
 * dst[k][b] = src[k][index[b]] for b < B, rows of row_bytes[k] bytes (a
 * multiple of 4), all in one launch.  An index outside [0, n_src) yields a
 * zero row (it is never dereferenced).  index is int64 (torch.randperm's
 * dtype).  PPO_ERR_TOO_LARGE when a combined row exceeds 2^30 words or
 * B times it exceeds 2^50.
 */
int ppo_gather_rows(const int64_t* index, int64_t B, int64_t n_src, int32_t narrays,
                    const void* const* src, const int32_t* row_bytes, void* const* dst,
                    void* stream);

/*
 * Host-to-device copy of nbytes (a multiple of 4, < 2 GiB) from pinned host
 * memory (hipHostMalloc / torch pin_memory) as one kernel launch on `stream`
 * that reads the pinned pages over the bus; no counterpart in the reference.
 * For the minibatch permutations of ppo.py:130, drawn on the CPU generator:
 * a small hipMemcpyAsync from the host can wait for the stream's earlier work
 * and stall the host, this launch does not.  The caller must keep src_host
 * unchanged until the stream has passed the launch.  Returns
 * PPO_ERR_INVALID_ARG (launching nothing) for memory that is not pinned and
 * mapped for the device.
 */
int ppo_copy_from_pinned(void* dst, const void* src_host, int64_t nbytes, void* stream);

/*
 * Batched action selection of PPOAgent.select_action (rl/deep/agents/ppo.py:
 * 65-79: Categorical(logits=policy(obs)).sample(), .log_prob(action),
 * value(obs)) for N environments at once, written straight into row t of a
 * [T,N] rollout buffer by passing pointers to that row.  For row n of
 * logits [N,A] and the caller's uniform u_n in [0,1):
 *   actions_out[n] = min{ j : u_n < sum_{k<=j} softmax(logits[n])_k }
 *                    (inverse CDF; A-1 if rounding leaves u_n above the total)
 *   logp_out[n]    = log softmax(logits[n])[actions_out[n]]
 *   values_out[n]  = values[n]            (skipped when either is NULL)
 * actions_out is int32.  Uniforms come from the caller (e.g. torch.rand on
 * the device with a seeded generator), so a rollout is reproducible.  No
 * workspace; no host synchronisation.
 */
int ppo_sample_cat_f32(const float* logits, int64_t N, int32_t A, const float* uniforms,
                       int32_t* actions_out, float* logp_out, const float* values,
                       float* values_out, void* stream);

/*
 * The continuous counterpart (Normal(mu, exp(log_std)).sample() and
 * .log_prob(action).sum(-1)) for the Gaussian policy: with the caller's
 * standard normals eps [N,D],
 *   actions_out[n,d] = mu[n,d] + exp(log_std[d]) * eps[n,d]
 *   logp_out[n]      = sum_d -(a-mu)^2/(2 sigma_d^2) - log sigma_d - log sqrt(2 pi)
 *   values_out[n]    = values[n]          (skipped when either is NULL)
 * D <= 24.
 */
int ppo_sample_gauss_f32(const float* mu, const float* log_std, int64_t N, int32_t D,
                         const float* normals, float* actions_out, float* logp_out,
                         const float* values, float* values_out, void* stream);

#define PPO_ADAM_MAX_TENSORS 32

typedef struct ppo_adam_params {
  double lr, beta1, beta2, eps;  /* torch.optim.Adam(lr, betas=(beta1, beta2), eps) */
  double max_grad_norm;          /* clip_grad_norm_ max_norm; <= 0: no clipping    */
  int64_t step;                  /* the step number after this update (>= 1)      */
  /* Optional device counter (NULL: use `step`).  When set, the first kernel
     increments *step_counter and the second derives the bias corrections from
     it on the device, so the call can be captured once in a graph and
     replayed for every step. */
  int64_t* step_counter;
} ppo_adam_params;

size_t ppo_adam_clip_workspace_bytes(int32_t ntensors, const int64_t* numel);

/*
 * Replaces nn.utils.clip_grad_norm_(params, max_grad_norm) + Adam.step()
 * (rl/deep/agents/ppo.py:170-171; TrainingConfig.lr, PPOConfig.gradient_clip)
 * for ntensors <= PPO_ADAM_MAX_TENSORS fp32 tensors: total norm of all
 * gradients (the norm of the per-tensor norms), grads *= min(max_norm /
 * (norm + 1e-6), 1) in place, then Adam (no weight decay, no amsgrad) on
 * params, exp_avg and exp_avg_sq in place, following torch's multi-tensor Adam
 * operation by operation in fp32.  grad_norm_out (may be NULL) receives the
 * total norm (clip_grad_norm_'s return value).  The pointer arrays are host
 * arrays of device pointers.
 */
int ppo_adam_clip_f32(int32_t ntensors, float* const* params, float* const* grads,
                      float* const* exp_avg, float* const* exp_avg_sq, const int64_t* numel,
                      const ppo_adam_params* hp, float* grad_norm_out, void* workspace,
                      size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Fused minibatch gradient through the actor and critic MLPs.              */
/* ------------------------------------------------------------------------ */

#define PPO_ACT_RELU 0  /* nn.ReLU (the reference's MLP, common.py:21-24)     */
#define PPO_ACT_TANH 1  /* nn.Tanh                                           */

/*
 * One MLP of rl/deep/agents/common.py:16-28, Linear(in,H)-act-Linear(H,H)-
 * act-Linear(H,out): weight[l] and bias[l] are the nn.Linear parameters of
 * layer l ([out,in] row-major fp32, 16-byte aligned weights); weight_grad[l]
 * and bias_grad[l] receive their gradients (same shapes, overwritten).
 */
typedef struct ppo_mlp3_f32 {
  const float* weight[3];
  const float* bias[3];
  float* weight_grad[3];
  float* bias_grad[3];
} ppo_mlp3_f32;

size_t ppo_mlp_cat_grad_workspace_bytes(int64_t B, int32_t obs_dim, int32_t hidden, int32_t A);

/*
 * Replaces the forward and backward of PPOAgent._update_batch (rl/deep/agents/
 * ppo.py:141-169) for one minibatch, from the observation rows to the
 * parameter gradients, together with the minibatch gather of ppo.py:132-139:
 *   rows      = index[0..B) (NULL: rows 0..B-1) of the [n, ...] arrays
 *   values    = critic(observations[rows]).squeeze(1)          (ppo.py:147)
 *   logits    = actor(observations[rows])                      (ppo.py:149)
 *   loss      = ppo_loss_cat_f32's loss over the B rows        (ppo.py:150-167)
 *   loss.backward()                                             (ppo.py:169)
 * writing the gradient of every actor and critic weight and bias (actor
 * output A logits, critic output 1; both hidden size `hidden`, one activation)
 * and scalars_out[PPO_NUM_SCALARS].  Requires obs_dim <= 64, A <= 32 and
 * hidden in {16, 32, 64, 128} (else PPO_ERR_UNSUPPORTED).  Gradients are
 * summed over the minibatch per 16-row workgroup and then across workgroups in
 * a fixed order (deterministic).  Follow with ppo_adam_clip_f32 for
 * clip_grad_norm_ + Adam (ppo.py:170-171).
 */
int ppo_mlp_cat_grad_f32(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic,
                         int32_t obs_dim, int32_t hidden, int32_t A, int32_t activation,
                         const float* observations, int64_t n, const int64_t* index, int64_t B,
                         const void* actions, int actions_are_int64,
                         const float* old_log_probs, const float* advantages,
                         const float* returns, const float* old_values,
                         const ppo_loss_params* params, float* scalars_out, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * A whole minibatch step of PPOAgent._update_batch (rl/deep/agents/
 * ppo.py:141-171): ppo_mlp_cat_grad_f32's gradients, then
 * clip_grad_norm_(max_grad_norm) + Adam as ppo_adam_clip_f32 over the 12
 * tensors in the order actor weight[0], bias[0], weight[1], bias[1],
 * weight[2], bias[2], then the critic's (the order of
 * list(policy.parameters()) + list(value.parameters())).  exp_avg and
 * exp_avg_sq are host arrays of 12 device pointers in that order; the
 * weights and biases of both structs are updated in place (so they must be
 * writable), their gradients hold the clipped gradients afterwards.  Two
 * launches: the gradient kernel, then one kernel that sums the gradient
 * partials, forms the clip norm and applies Adam (its workgroups wait for
 * each other, so it runs only when its grid fits on the device at once;
 * otherwise, or with PPO_AMD_MLP_FUSED_ADAM=0 in the environment, the sums
 * and the update are two launches, with bit-identical results).
 * adam->step_counter, when set, is incremented once.  grad_norm_out (may be
 * NULL) receives the total norm.  Same limits and workspace as
 * ppo_mlp_cat_grad_f32.
 */
int ppo_mlp_cat_step_f32(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic,
                         int32_t obs_dim, int32_t hidden, int32_t A, int32_t activation,
                         const float* observations, int64_t n, const int64_t* index, int64_t B,
                         const void* actions, int actions_are_int64, const float* old_log_probs,
                         const float* advantages, const float* returns, const float* old_values,
                         const ppo_loss_params* params, float* const* exp_avg,
                         float* const* exp_avg_sq, const ppo_adam_params* adam,
                         float* scalars_out, float* grad_norm_out, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * PPOAgent.select_action (rl/deep/agents/ppo.py:65-79) for N observations
 * through the actor and critic MLPs of ppo_mlp_cat_grad_f32 (only the weights
 * and biases of the structs are read): logits = actor(obs), values =
 * critic(obs), then ppo_sample_cat_f32's inverse-CDF draw at uniforms[n].
 * Writes actions_out (int32), log_probs_out and values_out, and copies the
 * observations to observations_out when it is not NULL (a rollout buffer
 * row).  One launch; same size limits as ppo_mlp_cat_grad_f32.
 */
int ppo_mlp_act_cat_f32(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic,
                        int32_t obs_dim, int32_t hidden, int32_t A, int32_t activation,
                        const float* observations, int64_t N, const float* uniforms,
                        float* observations_out, int32_t* actions_out, float* log_probs_out,
                        float* values_out, void* stream);

/*
 * The forward half of PPOAgent.select_action (ppo.py:65-79, lines 66 and
 * 73-77): logits_out [N,A] = actor(obs) and values_out [N] = critic(obs)
 * through the networks of ppo_mlp_cat_grad_f32, in one launch, so that a
 * caller sampling on the host (the reference's CPU Categorical, which
 * consumes torch's global generator) copies both back to the host at once.
 * observations, logits_out and values_out may be device memory or pinned
 * host memory (hipHostMalloc, torch pin_memory): the kernel then reads and
 * writes the host memory over the bus, and the caller reads the results
 * after synchronising the stream, with no copy launched.  Same size limits
 * as ppo_mlp_cat_grad_f32.
 */
int ppo_mlp_forward_cat_f32(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic,
                            int32_t obs_dim, int32_t hidden, int32_t A, int32_t activation,
                            const float* observations, int64_t N, float* logits_out,
                            float* values_out, void* stream);

/* ------------------------------------------------------------------------ */
/* Vectorised CartPole-v1 (the reference's environment, rl/deep/cli.py:    */
/* 179-180, stepped by rl/deep/runner.py:56-74).                            */
/* ------------------------------------------------------------------------ */

/*
 * Reset N environments: state[n] = -0.05 + 0.1 * uniforms[n] (fp64 [N,4]
 * from the caller's U[0,1) fp32 [N,4]), steps[n] = 0, obs_out = (float)state.
 */
int ppo_cartpole_reset(double* state, int32_t* steps, const float* uniforms, float* obs_out,
                       int64_t N, void* stream);

/*
 * One env.step(action) for N environments (gymnasium CartPoleEnv dynamics,
 * fp64, explicit Euler, tau 0.02; see csrc/cartpole.hip): actions int32 (1
 * pushes right); rewards_out = 1; dones_out = terminated (|x| > 2.4 or
 * |theta| > 12 deg) or truncated (steps reach max_steps, 500 for v1);
 * terminated_out (may be NULL) = terminated alone.  A done environment is
 * reset in the same launch from reset_uniforms [N,4] and obs_out holds its
 * reset observation.  Episode tally (all three NULL, or all set):
 * episode_return[n] accumulates the rewards of the running episode; when it
 * ends, its return is added to completed_sum[n] (fp64), completed_count[n]
 * is incremented and episode_return[n] restarts at 0.  No counterpart in the
 * reference's own code (its environment comes from gymnasium); no workspace.
 */
int ppo_cartpole_step(double* state, int32_t* steps, const int32_t* actions,
                      const float* reset_uniforms, int32_t max_steps, float* obs_out,
                      float* rewards_out, uint8_t* dones_out, uint8_t* terminated_out,
                      float* episode_return, double* completed_sum, int32_t* completed_count,
                      int64_t N, void* stream);

/*
 * A whole rollout of T steps for N CartPole environments in one launch: per
 * step, ppo_mlp_act_cat_f32 (actor 4-H-H-2, critic 4-H-H-1; only weights and
 * biases are read) at action_uniforms[t * action_uniforms_stride + n], then
 * ppo_cartpole_step with reset_uniforms[t * reset_uniforms_stride + 4n ..],
 * writing rollout buffer rows t: obs_buf [T,N,4] (the observation acted on),
 * actions_buf int32 [T,N], log_probs_buf, values_buf, rewards_buf [T,N] and
 * dones_buf uint8 [T,N].  observations [N,4] are the current observations;
 * observations_out (may equal observations) receives those after the last
 * step; state, steps and the episode tally (as ppo_cartpole_step, all three
 * NULL or all set) are updated in place.  The results equal T pairs of
 * ppo_mlp_act_cat_f32 + ppo_cartpole_step launches on the same uniforms.
 * Replaces the per-step loop of rl/deep/runner.py:56-74 (select_action,
 * env.step, the agent's rollout append) for N environments; no workspace.
 */
int ppo_cartpole_rollout_f32(const ppo_mlp3_f32* actor, const ppo_mlp3_f32* critic,
                             int32_t hidden, int32_t activation, int64_t N, int32_t T,
                             int32_t max_steps, double* state, int32_t* steps,
                             const float* observations, float* observations_out,
                             const float* action_uniforms, int64_t action_uniforms_stride,
                             const float* reset_uniforms, int64_t reset_uniforms_stride,
                             float* obs_buf, int32_t* actions_buf, float* log_probs_buf,
                             float* values_buf, float* rewards_buf, uint8_t* dones_buf,
                             float* episode_return, double* completed_sum,
                             int32_t* completed_count, void* stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* PPO_AMD_H */
