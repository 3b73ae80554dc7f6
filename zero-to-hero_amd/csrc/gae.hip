// Generalized advantage estimation over an env-contiguous [T,N] rollout.
//
// Reference: PPOAgent._advantages, rl/deep/agents/ppo.py:173-193, plus
// `returns = advantages + old_values` (ppo.py:124).  The reference walks one
// episode backwards in Python floats:
//     mask  = 1 - float(terminated or truncated)                   (:179)
//     delta = reward + gamma*next_value*mask - value               (:180-184)
//     adv   = delta + gamma*lambda*mask*adv                        (:185-188)
//     next_value = value                                           (:190)
// Every thread here performs that recurrence in fp64 with the same operation
// order and no fused multiply-adds, so an element whose carry is exact is
// bit-identical to the reference after the final fp32 cast.
//
// Parallel structure (HBM-streaming kernels):
//   The recurrence is affine in the carried advantage: adv_t = delta_t +
//   c_t*adv_{t+1} with c_t = gamma*lambda*mask_t.  A run of steps therefore
//   maps the advantage entering it from the right, x, to a + P*x.
//   * A "segment" is L consecutive steps of VW adjacent envs owned by one
//     thread (VW=4: float4 row loads, dones read as one 32-bit word).
//   * A "tile" is Sw consecutive segments x Qw adjacent env-groups owned by
//     one 256-thread workgroup; segments are composed by lane shuffles in each
//     wave and a fold of the four waves in LDS.
//   1. gae_tile_kernel<kSummary>: per tile and env, the composite (a, P) of
//      all its steps -> workspace `summary` [Tt][N].
//   2. gae_carry_kernel: per env, a reverse scan over the tiles' (a, P) ->
//      `carry` [Tt][N], the advantage entering each tile from the right
//      (two levels, via per-chunk composites, for long horizons).
//   3. gae_tile_kernel<kFinal>: re-reads the tile, rebuilds the
//      segment composites, applies the tile carry, and runs the exact serial
//      recurrence per segment, writing adv and ret.
// Fused normalisation (ppo_gae_norm_f32): the final pass also leaves per-block
// fp64 (n, sum, sum of squares) of its fp32 advantages, and the elementwise
// normaliser runs after it.  When the whole horizon fits in one tile (Tt ==
// 1) steps 1-2 are skipped.
//
// Wide rollouts (N >= 2048, aligned) take a single-pass "strip walk" instead
// (gae_strip_kernel): a workgroup owns 8-32 adjacent envs for the whole
// horizon and walks it backwards in chunks, carrying the advantage from chunk
// to chunk, so the rollout is read once; the normaliser then needs one
// elementwise pass over the advantages.
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "grid_sync.hpp"
#include "stats.hpp"

namespace ppo {
namespace {

struct GaeArgs {
  const float* r;
  const float* v;
  const uint8_t* d;
  const float* lastv;  // may be null (zeros)
  // v may be null (all values zero: discounted returns, the REINFORCE case)
  long T, N;
  double gamma, gl;    // gamma and gamma*lambda (the product rounded once, as in Python)
  float* adv;
  float* ret;          // may be null
  double2* summary;    // [Tt][N] (a, P)
  double2* chunk_sum;  // [nchunks][N] (a, P) of each carry-scan chunk
  const double* carry; // [Tt][N] or null (all-zero carries)
  double* partial;     // [.][4] (n, sum, sum sq) partials of the advantages
  float* adv_n;        // normalised advantages
  WsHeader* hdr;
  float* stats_out;
  double eps;
  long Q, Tq, Tt, span;
  int Qw, Sw;
  long nstrips, spans, span_tiles;  // span passes: env strips, spans per strip, tiles per span
  uint64_t* slots;     // resident pass: barrier counter, tile composites, per-workgroup partials
  unsigned nonce;      // resident pass: tag of this call in the barrier counter
  long res_nc, res_nt; // resident pass: env columns, time tiles
  long res_ntr, res_rounds;  // resident pass: time tiles per round, rounds
  WaitCtl wc;          // resident pass: poll limit and the device's wait-status word
};

// What a gae_tile_kernel launch computes.
enum GaeMode {
  kSummary = 0,       // pass 1: tile composites
  kFinal = 2,         // pass 2: adv, ret
  kFinalPartials = 3, // pass 2: adv, ret + per-block fp64 (n, sum, sum sq) for the normaliser
};

// Geometry of one tile pass: L steps x VW envs per thread, Sw segments x Qw
// env-groups per 256-thread tile (Sw * L steps), Tq tiles across the envs.
struct PassGeom {
  int L, Qw, Sw;
  long Tq;
  bool solo;  // Sw == 1: the thread's segment is the tile, no LDS scan
};

struct GaePlan {
  long T;
  int vw;
  long Q, Tt, span;
  PassGeom scan, fin;  // pass 1 (tile composites) and the final pass
  PassGeom fin_solo;   // final pass without the normaliser (wide rollouts only)
  long blocks() const { return Tt * std::max(std::max(scan.Tq, fin.Tq), fin_solo.Tq); }
  // the final pass's geometry: solo tiles where they exist and no normaliser
  const PassGeom& final_geom(bool norm) const { return !norm && fin_solo.Tq > 0 ? fin_solo : fin; }
};

PassGeom make_geom(long Q, int L, int Qw) {
  PassGeom g;
  g.L = L;
  g.Qw = Qw;
  g.Sw = kBlock / Qw;
  g.Tq = (Q + Qw - 1) / Qw;
  g.solo = g.Sw == 1;
  return g;
}


// Tiles span 16 steps for VW = 4 and 256/Qw * 16 steps for VW = 1.  Narrow
// rollouts stack Sw = 256/Qw segments per tile (Qw <= 64 env-groups) and
// compose them with an LDS scan, keeping a workgroup's rows wide enough to
// coalesce.  Wide rollouts (VW = 4, >= 256 env-groups) have 4 segments of 4
// steps x 64 env-groups per tile; their final pass without the normaliser
// takes solo tiles instead, chosen by measurement at T=2048, N=4096 (kernel
// us, stacked / solo): pass 1 17.9 / -, final pass 26.6 / 23.0.
// (solo tiles are 16 steps x 4 envs per thread, 256 env-groups per tile: the
// same tile boundaries in T, so their carries are interchangeable.)
GaePlan make_plan(long T, long N, int vw) {
  GaePlan p;
  p.T = T;
  p.vw = vw;
  p.Q = N / vw;
  p.fin_solo.Tq = 0;
  if (vw == 1) {
    const int Qw = (int)std::min<long>(64, (long)pow2_ceil((unsigned)std::min<long>(p.Q, 64)));
    p.scan = p.fin = make_geom(p.Q, 16, Qw);
  } else if (p.Q < kBlock) {
    const int Qw = (int)std::min<long>(64, (long)pow2_ceil((unsigned)std::min<long>(p.Q, 64)));
    p.scan = p.fin = make_geom(p.Q, 4, Qw);
  } else {
    p.scan = make_geom(p.Q, 4, 64);
    p.fin = make_geom(p.Q, 4, 64);
    p.fin_solo = make_geom(p.Q, 16, kBlock);
  }
  p.span = (long)p.fin.Sw * p.fin.L;
  p.Tt = (T + p.span - 1) / p.span;
  return p;
}

// Carry-scan geometry (see gae_carry_kernel): 1024-thread blocks of Ew envs x
// Rw rows, 8 tile composites per thread, so a chunk spans Rw*8 tiles.
constexpr int kCarryBlock = 1024;
constexpr int kCarryG = 8;

struct CarryPlan {
  int Ew, Rw;
  long groups, nchunks;
};

// Ew envs per block (16-64, for 128-512-byte coalesced summary rows), halved
// down to 16 until the envs alone give >= 256 blocks; Rw rows, no more than
// the horizon needs (G tiles per row), no more than fit 1024 threads, and at
// least one full wave per block.
CarryPlan make_carry_plan(long Tt, long N) {
  CarryPlan c;
  c.Ew = (int)std::min<long>(64, (long)pow2_ceil((unsigned)std::min<long>(N, 64)));
  while (c.Ew > 16 && (N + c.Ew - 1) / c.Ew < 256) c.Ew >>= 1;
  const long rows_needed = (Tt + kCarryG - 1) / kCarryG;
  c.Rw = (int)std::min<long>(kCarryBlock / c.Ew,
                             (long)pow2_ceil((unsigned)std::min<long>(rows_needed, 1024)));
  c.Rw = std::max(c.Rw, kWave / c.Ew);  // whole waves: block reductions assume them
  c.groups = (N + c.Ew - 1) / c.Ew;
  const long chunk_tiles = (long)c.Rw * kCarryG;
  c.nchunks = (Tt + chunk_tiles - 1) / chunk_tiles;
  return c;
}

// Strip-walk geometry (gae_strip_kernel): 1024-thread workgroups, each
// owning a strip of E envs (one env and kStripL consecutive steps per thread)
// for the whole horizon, in chunks of (1024/E)*kStripL steps.  E is the widest
// of 32, 16, 8 that still gives every CU a strip (kStripMinBlocks) and keeps
// at least a quarter of a chunk's threads busy; narrower rollouts, very short
// horizons, misaligned buffers and rollouts of >= 2^30 elements take the tile
// passes (measured: T=16, N=65536 runs 12 us tiled, 36 us as strips).
#ifndef PPO_GAE_STRIP_BLOCK
#define PPO_GAE_STRIP_BLOCK 1024
#endif
#ifndef PPO_GAE_STRIP_EMAX
#define PPO_GAE_STRIP_EMAX 32
#endif
#ifndef PPO_GAE_STRIP_L
#define PPO_GAE_STRIP_L 8
#endif
constexpr int kStripBlock = PPO_GAE_STRIP_BLOCK;
constexpr int kStripL = PPO_GAE_STRIP_L;
// (PPO_GAE_STRIP_MIN: build-time override, e.g. to time the tile passes alone)
#ifndef PPO_GAE_STRIP_MIN
#define PPO_GAE_STRIP_MIN 256
#endif
constexpr long kStripMinBlocks = PPO_GAE_STRIP_MIN;

struct StripPlan {
  int E;        // envs per strip (0: use the tile passes)
  long strips;  // workgroups
};

StripPlan strip_plan(const GaePlan& p) {
  const long T = p.T;
  StripPlan sp = {0, 0};
  const long N = p.Q * p.vw;
  if (p.vw != 4 || T * N >= (1L << 30)) return sp;
  for (int E = PPO_GAE_STRIP_EMAX; E >= 8; E >>= 1) {
    const long strips = (N + E - 1) / E;
    const long chunk = (long)(kStripBlock / E) * kStripL;
    if (strips >= kStripMinBlocks && 4 * T >= chunk) {
      sp.E = E;
      sp.strips = strips;
      return sp;
    }
  }
  return sp;
}

#ifndef PPO_GAE_SPAN
#define PPO_GAE_SPAN 1  // build-time switch: 0 keeps narrow rollouts on the tile passes
#endif
// Span geometry (gae_span_*_kernel): strips of E envs (the largest power of
// two <= 64 dividing N), time tiles of 16 * 256/E steps (4096 elements), and
// about `blocks` workgroups in all, each owning a span of `tps` consecutive
// tiles of one strip.
constexpr long kSpanMaxBlocks = 2048;

struct SpanPlan {
  int E;        // envs per strip (0: not applicable)
  long nstrips, tt, tps, spans;  // strips, time tiles, tiles per span, spans per strip
};

SpanPlan span_plan(long T, long N, long blocks) {
  SpanPlan c = {0, 0, 0, 0, 0};
  if (T <= 0 || N <= 0 || N % 4 != 0) return c;
  int E = 64;
  while (N % E != 0) E >>= 1;
  const long S = 16L * (256 / E);
  c.nstrips = N / E;
  c.tt = (T + S - 1) / S;
  const long per_strip = std::max(1L, std::min(c.tt, blocks / c.nstrips));
  c.tps = (c.tt + per_strip - 1) / per_strip;
  c.spans = (c.tt + c.tps - 1) / c.tps;
  if (c.nstrips * c.spans <= 0x7fffffffL) c.E = E;
  return c;
}

// Resident-pass geometry (gae_resident_kernel): 1024-thread workgroups, each
// owning a tile of E envs x TS = (1024/(E/4))*L steps (4 envs and L steps per
// thread) whose rows stay in registers from load to store.  The grid is one
// tile per workgroup and must be resident at once (checked at launch against
// the occupancy of the chosen kernel), so tiles can wait on each other.
// PPO_GAE_RES: build-time switch, 0 keeps every rollout on the other paths;
// PPO_GAE_RES_E: build-time choice of the tile width (0: by the plan).
#ifndef PPO_GAE_RES
#define PPO_GAE_RES 1
#endif
#ifndef PPO_GAE_RES_E
#define PPO_GAE_RES_E 0
#endif

#ifndef PPO_GAE_RES_BLOCK
#define PPO_GAE_RES_BLOCK 512
#endif
constexpr int kResBlock = PPO_GAE_RES_BLOCK;
constexpr long kResMaxTiles = 256;  // one workgroup per CU on MI355X

struct ResPlan {
  int E, L;          // E = 0: not applicable
  long nc, nt, TS;   // env columns, time tiles, steps per tile
  long ntr, rounds;  // time tiles per round (per column), rounds
  long grid() const { return nc * ntr; }
  long tiles() const { return nc * nt; }
};

// Single round: among tiles of 128 envs and 16 steps per thread, or 64, 32
// or 16 envs and 16, 8 or 4 steps per thread, the shape giving the most tiles
// that still fit on the device at once (<= 256), with no more than a quarter
// of a column's threads idle past the horizon; ties go to wider tiles (longer
// row segments: at T x N = 2048 x 4096 with the normaliser, 128-env tiles
// measured 38.2-38.5 us per call in the north-star step against 39.1-39.3 us
// for 64-env tiles; 256-env tiles were slower, their look-back folding 15
// tiles per column, so 128-env tiles are taken only up to 8 tiles per column).  Rollouts that
// give fewer than 128 tiles (too little parallelism), or more than 16 tiles
// per env column without filling the device, take the other paths: measured
// on MI355X, e.g. T x N = 1024 x 512 (16-64 tiles) 28 us against 24 us on the
// tile passes, while 2048 x 4096 runs 45 us against 55 us, 4096 x 2048 45 us
// against 72 and 32768 x 256 (64 tiles per column, 256 tiles) 57 us against 67.
// Without the normaliser, rollouts too long for one round (more than 256
// tiles of 16 steps per thread) run in rounds of 256 tiles, from the end of
// the horizon backwards (at most kResMaxRounds), each round handing the
// advantage at its left edge to the next.
constexpr long kResMaxRounds = 8;

ResPlan res_plan(long T, long N, bool norm) {
  ResPlan best = {0, 0, 0, 0, 0, 0, 0};
  if (!PPO_GAE_RES || T <= 0 || N <= 0 || T * N >= (1L << 30)) return best;
  const int Es[4] = {128, 64, 32, 16};
  const int Ls[3] = {16, 8, 4};
  for (int E : Es) {
    if (PPO_GAE_RES_E && E != PPO_GAE_RES_E) continue;
    if (N % E != 0) continue;
    for (int L : Ls) {
      if (E == 128 && L != 16) continue;  // (128-env tiles: 16 steps per thread only)
      const long TS = (long)(kResBlock / (E / 4)) * L;
      const long nt = (T + TS - 1) / TS;
      const long nc = N / E;
      if (nc * nt > kResMaxTiles) continue;
      if (E == 128 && nt > 8) continue;  // (a longer look-back than 64-env tiles')
      if (4 * (nt * TS - T) > nt * TS) continue;  // a quarter of the threads idle
      if (nc * nt > best.tiles()) {
        best.E = E;
        best.L = L;
        best.nc = nc;
        best.nt = nt;
        best.TS = TS;
        best.ntr = nt;
        best.rounds = 1;
      }
    }
  }
  if (best.E && (best.tiles() < 128 || (best.nt > 16 && best.tiles() < kResMaxTiles)))
    best.E = 0;
  if (best.E || norm) return best;
  // rounds: the widest tile of at most 64 envs dividing N, 16 steps per thread
  for (int E : Es) {
    if (E == 128) continue;
    if (PPO_GAE_RES_E && E != PPO_GAE_RES_E) continue;
    if (N % E != 0) continue;
    const long nc = N / E;
    if (nc > kResMaxTiles) continue;
    const long TS = (long)(kResBlock / (E / 4)) * 16;
    const long nt = (T + TS - 1) / TS;
    const long ntr = kResMaxTiles / nc;
    const long rounds = (nt + ntr - 1) / ntr;
    if (rounds < 2 || rounds > kResMaxRounds) continue;
    if (4 * (nt * TS - T) > nt * TS) continue;
    best.E = E;
    best.L = 16;
    best.nc = nc;
    best.nt = nt;
    best.TS = TS;
    best.ntr = ntr;
    best.rounds = rounds;
    return best;
  }
  return best;
}

// 64-bit slot words of the resident pass: the start barrier's counter (a
// block of 32 words), per tile E composites (a, P) of two words each, per
// round one carry per env (the advantage at the round's left edge), then
// three words (n, sum, sum of squares) per workgroup.
constexpr size_t kResSlotBase = kSyncWords;
// per workgroup: n, sum and sum of squares of its advantages, and the centred
// sum of squares of the exact second pass (gae_resident_kernel, step 4)
constexpr size_t kResPartWords = 4;
size_t res_slot_words(const ResPlan& rp) {
  if (!rp.E) return 0;
  return kResSlotBase + (size_t)rp.tiles() * 2 * rp.E + (size_t)rp.rounds * rp.nc * rp.E +
         (size_t)rp.grid() * kResPartWords;
}
size_t res_slot_words_max(long T, long N) {
  return std::max(res_slot_words(res_plan(T, N, true)), res_slot_words(res_plan(T, N, false)));
}

struct GaeLayout {
  size_t summary, carry, chunk_sum, partial, slots, total;
};

GaeLayout make_layout(const GaePlan& p, long N) {
  GaeLayout l;
  size_t off = kHeaderBytes;
  l.summary = off;  // tile composites [Tt][N], or the span composites [spans][N]
  {
    const SpanPlan sp = span_plan(p.T, N, kSpanMaxBlocks);
    off += align_up(std::max<size_t>((size_t)p.Tt * N, (size_t)sp.spans * N) * sizeof(double2), 256);
  }
  const long ncarry = std::max(p.Tt, span_plan(p.T, N, kSpanMaxBlocks).spans);
  l.carry = off;
  off += align_up((size_t)ncarry * N * sizeof(double), 256);
  l.chunk_sum = off;
  off += align_up((size_t)std::max(make_carry_plan(p.Tt, N).nchunks,
                                   make_carry_plan(ncarry, N).nchunks) * N * sizeof(double2), 256);
  l.partial = off;
  {
    const CarryPlan cp = make_carry_plan(p.Tt, N);
    const SpanPlan sp = span_plan(p.T, N, kSpanMaxBlocks);
    const long parts = std::max<long>(std::max<long>(p.blocks(), cp.groups * cp.nchunks),
                                      std::max<long>(strip_plan(p).strips, sp.nstrips * sp.spans));
    off += align_up((size_t)parts * 4 * sizeof(double), 256);
  }
  l.slots = off;
  off += align_up(res_slot_words_max(p.T, N) * sizeof(uint64_t), 256);
  l.total = off;
  return l;
}

// fp64 multiply / add with no contraction into FMA: the reference evaluates
// each Python float operation with its own rounding.  (HIP's __dmul_rn /
// __dadd_rn are plain operators that the backend may still fuse; the pragma
// takes the contraction flag off these operations themselves.)
__device__ __forceinline__ double mul(double a, double b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ double add(double a, double b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ double sub(double a, double b) {
#pragma clang fp contract(off)
  return a - b;
}

// Rollout arrays are streamed: nontemporal loads and stores.
typedef float f4 __attribute__((ext_vector_type(4)));

#ifndef PPO_GAE_NT_LOAD
#define PPO_GAE_NT_LOAD 0
#endif
#ifndef PPO_GAE_NT_STORE
#define PPO_GAE_NT_STORE 1
#endif
template <typename T>
__device__ __forceinline__ T ld(const T* p) {
  if constexpr (PPO_GAE_NT_LOAD) return __builtin_nontemporal_load(p);
  else return *p;
}
template <typename T>
__device__ __forceinline__ void st(T v, T* p) {
  if constexpr (PPO_GAE_NT_STORE) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <int VW>
__device__ __forceinline__ void load_f(const float* p, float (&x)[VW]) {
  if constexpr (VW == 4) {
    const f4 t = ld(reinterpret_cast<const f4*>(p));
    x[0] = t[0]; x[1] = t[1]; x[2] = t[2]; x[3] = t[3];
  } else {
    x[0] = ld(p);
  }
}

template <int VW>
__device__ __forceinline__ void store_f(float* p, const float (&x)[VW]) {
  if constexpr (VW == 4) {
    const f4 t = {x[0], x[1], x[2], x[3]};
    st(t, reinterpret_cast<f4*>(p));
  } else {
    st(x[0], p);
  }
}

typedef float f2 __attribute__((ext_vector_type(2)));
template <int VW>
__device__ __forceinline__ void load_vec(const float* p, float (&x)[VW]) {
  if constexpr (VW == 2) {
    const f2 t = ld(reinterpret_cast<const f2*>(p));
    x[0] = t[0]; x[1] = t[1];
  } else {
    load_f<VW>(p, x);
  }
}
// Plain (temporal) stores: the strip walk writes half cache lines from two
// workgroups on the same XCD, which the L2 merges only if it holds them
// (with nontemporal stores the HBM writes measured 1.33x the bytes).
template <int VW>
__device__ __forceinline__ void store_vec(float* p, const float (&x)[VW]) {
  if constexpr (VW == 4) {
    *reinterpret_cast<f4*>(p) = f4{x[0], x[1], x[2], x[3]};
  } else if constexpr (VW == 2) {
    *reinterpret_cast<f2*>(p) = f2{x[0], x[1]};
  } else {
    *p = x[0];
  }
}

// Nontemporal form, for stores that cover whole 128-byte lines.
template <int VW>
__device__ __forceinline__ void store_vec_nt(float* p, const float (&x)[VW]) {
  static_assert(VW == 4, "nontemporal stores are used for 16-byte pieces");
  __builtin_nontemporal_store(f4{x[0], x[1], x[2], x[3]}, reinterpret_cast<f4*>(p));
}

// Returns one bit per env: bit k set when dones[.., env0+k] != 0.
template <int VW>
__device__ __forceinline__ unsigned load_done(const uint8_t* p) {
  if constexpr (VW == 4) {
    const unsigned w = ld(reinterpret_cast<const unsigned*>(p));
    return ((w & 0xffu) != 0u) | (((w >> 8) & 0xffu) != 0u) << 1 |
           (((w >> 16) & 0xffu) != 0u) << 2 | ((w >> 24) != 0u) << 3;
  } else {
    return ld(p) != 0;
  }
}

// The done bytes of VW envs as loaded (byte k: env k), tested where used:
// inspecting them at load time makes the compiler wait for the load there.
template <int VW>
__device__ __forceinline__ unsigned load_done_raw(const uint8_t* p) {
  if constexpr (VW == 4) return ld(reinterpret_cast<const unsigned*>(p));
  else if constexpr (VW == 2) return ld(reinterpret_cast<const unsigned short*>(p));
  else return ld(p);
}

// Tile layouts: how a tile's Sw segments map to the workgroup's threads.
enum TileLayout {
  kStacked = 0,  // segment s of env-group q is thread s*Qw + q; LDS scan across waves
  kSoloTile = 1, // Sw == 1: the thread's segment is the tile
};

template <int VW, int L, int kLayout, int kMode>
__global__ void __launch_bounds__(kBlock) gae_tile_kernel(GaeArgs a) {
  constexpr bool kLds = kLayout == kStacked;
  constexpr bool kIsFinal = kMode >= kFinal;
  __shared__ double s_a[kLds ? kBlock * VW : 1];
  __shared__ double s_p[kLds ? kBlock * VW : 1];

  const long bid = blockIdx.x;
  const long tile_t = bid / a.Tq;
  const long tile_q = bid - tile_t * a.Tq;
  const int tid = threadIdx.x;
  const int q = tid % a.Qw;
  const int s = tid / a.Qw;
  const long col = tile_q * a.Qw + q;
  const bool col_ok = col < a.Q;
  const long env0 = col * VW;
  const long t0 = (tile_t * a.Sw + s) * (long)L;
  const long remain = a.T - t0;
  const int nvalid = col_ok ? (int)(remain <= 0 ? 0 : (remain < L ? remain : L)) : 0;

  // Loads are unconditional (rows past the horizon or the last env re-read
  // element 0 and are never used; absent values / bootstrap read the rewards
  // and are replaced by zeros where used): a load under a branch makes the
  // compiler wait for every load in flight at the join.
  float r[L][VW], v[L][VW], nv[VW];
  unsigned draw[L];
  const bool has_v = a.v != nullptr;
  const float* vsrc = has_v ? a.v : a.r;
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const long off = i < nvalid ? (t0 + i) * a.N + env0 : 0;
    load_f<VW>(a.r + off, r[i]);
    load_f<VW>(vsrc + off, v[i]);
    draw[i] = load_done_raw<VW>(a.d + off);
  }
  {
    const bool inner = t0 + L < a.T;
    float nvn[VW], nvl[VW];
    load_f<VW>(vsrc + ((nvalid > 0 && inner) ? (t0 + L) * a.N + env0 : 0), nvn);
    load_f<VW>((a.lastv ? a.lastv : a.r) + (col_ok ? env0 : 0), nvl);
#pragma unroll
    for (int k = 0; k < VW; ++k)
      nv[k] = inner ? (has_v ? nvn[k] : 0.0f) : (a.lastv ? nvl[k] : 0.0f);
  }
  auto val = [&](int i, int k) { return has_v ? v[i][k] : 0.0f; };
  auto isdone = [&](int i, int k) {
    if constexpr (VW == 1) return draw[i] != 0u;
    else return ((draw[i] >> (8 * k)) & 0xffu) != 0u;
  };

  // Composite (a, P) of this segment with a zero carry.
  double ia[VW], ip[VW];
  {
    double nvd[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      ia[k] = 0.0; ip[k] = 1.0; nvd[k] = nv[k];
    }
#pragma unroll
    for (int i = L - 1; i >= 0; --i) {
      if (i < nvalid) {
#pragma unroll
        for (int k = 0; k < VW; ++k) {
          const double m = isdone(i, k) ? 0.0 : 1.0;
          const double vd = (double)val(i, k);
          const double delta = sub(add((double)r[i][k], mul(mul(a.gamma, nvd[k]), m)), vd);
          const double c = mul(a.gl, m);
          ia[k] = add(delta, mul(c, ia[k]));
          ip[k] = mul(ip[k], c);
          nvd[k] = vd;
        }
      }
    }
  }

  // Reverse scan over the Sw segments of the tile (solo tiles: the segment is
  // the tile).  Stacked tiles: reverse scan of the segments inside each wave
  // by lane moves (segment s + 1 is lane + Qw), the four
  // waves' composites through LDS (one barrier), then each segment's
  // exclusive composite (of the segments after it) = its wave's exclusive
  // part followed by the later waves.  (ex_a, ex_p) is the identity for the
  // tile's last segment; tile_a/tile_p is the whole tile (segment 0).
  constexpr bool kWaveScan = kLds;
  double ex_a[VW], ex_p[VW], tile_a[VW], tile_p[VW];
  if constexpr (kWaveScan) {
    constexpr int kWaves = kBlock / kWave;
    const int lane = tid % kWave;
    const int w = tid / kWave;
    const int SW = kWave / a.Qw;     // segments per wave
    const int js = lane / a.Qw;      // this segment's index in its wave
    for (int off = 1; off < SW; off <<= 1) {
#pragma unroll
      for (int k = 0; k < VW; ++k) {
        const double pa = __shfl_down(ia[k], off * a.Qw);
        const double pp = __shfl_down(ip[k], off * a.Qw);
        if (js + off < SW) {
          ia[k] = ia[k] + ip[k] * pa;
          ip[k] = ip[k] * pp;
        }
      }
    }
    if (js == 0) {
#pragma unroll
      for (int k = 0; k < VW; ++k) {
        s_a[(w * a.Qw + q) * VW + k] = ia[k];
        s_p[(w * a.Qw + q) * VW + k] = ip[k];
      }
    }
    double na[VW], np[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      na[k] = __shfl_down(ia[k], a.Qw);
      np[k] = __shfl_down(ip[k], a.Qw);
      if (js + 1 >= SW) {
        na[k] = 0.0;
        np[k] = 1.0;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      double la = 0.0, lp = 1.0;  // the waves after this one, composed
      for (int ww = kWaves - 1; ww > w; --ww) {
        const double wa = s_a[(ww * a.Qw + q) * VW + k], wp = s_p[(ww * a.Qw + q) * VW + k];
        la = wa + wp * la;
        lp = wp * lp;
      }
      ex_a[k] = na[k] + np[k] * la;
      ex_p[k] = np[k] * lp;
      tile_a[k] = ia[k] + ip[k] * la;
      tile_p[k] = ip[k] * lp;
    }
  }
  if constexpr (!kIsFinal) {
    if (s == 0 && col_ok) {
#pragma unroll
      for (int k = 0; k < VW; ++k)
        a.summary[tile_t * a.N + env0 + k] =
            kWaveScan ? make_double2(tile_a[k], tile_p[k]) : make_double2(ia[k], ip[k]);
    }
    return;
  } else {
    // Advantage entering this segment from the right.
    double cin[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      const double C = (a.carry && col_ok) ? a.carry[tile_t * a.N + env0 + k] : 0.0;
      cin[k] = kWaveScan ? ex_a[k] + ex_p[k] * C : C;
    }

    // Exact serial recurrence over the segment; r[][] is reused for adv.
    {
      double adv[VW], nvd[VW];
#pragma unroll
      for (int k = 0; k < VW; ++k) { adv[k] = cin[k]; nvd[k] = nv[k]; }
#pragma unroll
      for (int i = L - 1; i >= 0; --i) {
        if (i < nvalid) {
#pragma unroll
          for (int k = 0; k < VW; ++k) {
            const double m = isdone(i, k) ? 0.0 : 1.0;
            const double vd = (double)val(i, k);
            const double delta = sub(add((double)r[i][k], mul(mul(a.gamma, nvd[k]), m)), vd);
            adv[k] = add(delta, mul(mul(a.gl, m), adv[k]));
            r[i][k] = (float)adv[k];
            nvd[k] = vd;
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < L; ++i) {
      if (i < nvalid) {
        const long off = (t0 + i) * a.N + env0;
        store_f<VW>(a.adv + off, r[i]);
        if (a.ret) {
          float rt[VW];
#pragma unroll
          for (int k = 0; k < VW; ++k) rt[k] = r[i][k] + val(i, k);
          store_f<VW>(a.ret + off, rt);
        }
      }
    }

    if constexpr (kMode == kFinalPartials) {
      double acc[3] = {(double)(nvalid * VW), 0.0, 0.0};
#pragma unroll
      for (int i = 0; i < L; ++i)
        if (i < nvalid)
#pragma unroll
          for (int k = 0; k < VW; ++k) {
            const double x = (double)r[i][k];
            acc[1] += x;
            acc[2] += x * x;
          }
      block_sum<3>(acc);
      if (tid == 0) {
        a.partial[bid * 4 + 0] = acc[0];
        a.partial[bid * 4 + 1] = acc[1];
        a.partial[bid * 4 + 2] = acc[2];
        a.partial[bid * 4 + 3] = 0.0;
      }
    }
  }
}

// Reverse scan of tile composites into per-tile carries, two levels.
// A "chunk" is kCarryChunk = Rw*G consecutive tiles of Ew envs, owned by one
// 1024-thread block: its Rw thread-rows hold G tile composites each in
// registers and are combined with a Kogge-Stone scan in LDS.
//   kCompose: each chunk's composite -> chunk_sum[c][env]        (many chunks only)
//   kCarry:   fold the composites of all later chunks (Rw at a time, scanned in
//             LDS) into the advantage entering this chunk, then scan the chunk
//             and write carry[k][env] for each of its tiles.
// Horizons of up to Rw*G tiles are one chunk and need only the kCarry launch.

// Reverse inclusive scan over the Rw thread-rows of (ga, gp) in LDS; returns
// with s_a/s_p holding, for row g, the composite of rows g..Rw-1.
// The product of two tiles' factor products, kept nonzero when neither is
// zero.  In the reference's serial recurrence an infinite advantage becomes
// NaN only by a zero factor (a done flag, or gamma * lambda = 0): it is
// multiplied by gamma * lambda once per step and never underflows.  Products
// composed over many tiles do underflow, and 0 x inf would then give NaN where
// the reference keeps the infinity; the smallest subnormal in place of such a
// zero keeps the infinity and changes no finite carry (its terms lie far below
// an ulp).  Used where tiles (spans, chunks) are composed: the carry scan, the
// span chain and the resident pass's look-back.  Inside a tile the products
// are plain (measured on the resident pass: 0.5-1.5 us per config-3 call on
// its critical path), so a tile's own product (gamma * lambda)^steps must not
// underflow for this to hold: gamma * lambda > 2^(-1074 / steps per tile),
// e.g. 0.70 for the resident pass's 2048-step tiles of 16 envs.
__device__ __forceinline__ double prod_nz(double x, double y) {
  const double p = x * y;
  return (p == 0.0 && x != 0.0 && y != 0.0) ? __builtin_copysign(4.9406564584124654e-324, p) : p;
}

__device__ __forceinline__ void carry_row_scan(double* s_a, double* s_p, int tid, int g, int Ew,
                                               int Rw, double ga, double gp) {
  s_a[tid] = ga;
  s_p[tid] = gp;
  for (int off = 1; off < Rw; off <<= 1) {
    __syncthreads();
    const bool has = g + off < Rw;
    double pa = 0.0, pp = 1.0;
    if (has) {
      pa = s_a[tid + off * Ew];
      pp = s_p[tid + off * Ew];
    }
    __syncthreads();
    if (has) {
      ga = ga + gp * pa;
      gp = prod_nz(gp, pp);
      s_a[tid] = ga;
      s_p[tid] = gp;
    }
  }
  __syncthreads();
}

template <bool kCompose>
__global__ void __launch_bounds__(kCarryBlock) gae_carry_kernel(const double2* __restrict__ summary,
                                                                 double* __restrict__ carry,
                                                                 double2* __restrict__ chunk_sum,
                                                                 long Tt, long N, int Ew, int Rw,
                                                                 long nchunks) {
  __shared__ double s_a[kCarryBlock];
  __shared__ double s_p[kCarryBlock];
  const int tid = threadIdx.x;
  const int e = tid % Ew;
  const int g = tid / Ew;
  const long env = (long)blockIdx.x * Ew + e;
  const bool ok = env < N;
  const long c = blockIdx.y;
  const long chunk_tiles = (long)Rw * kCarryG;
  const long lo = c * chunk_tiles;
  const long hi = lo + chunk_tiles < Tt ? lo + chunk_tiles : Tt;

  // advantage entering this chunk from the right
  double C = 0.0;
  if constexpr (!kCompose) {
    for (long top = nchunks; top > c + 1; top -= Rw) {
      const long bot = top - Rw > c + 1 ? top - Rw : c + 1;
      const long j = bot + g;
      double ga = 0.0, gp = 1.0;
      if (ok && j < top) {
        const double2 t = chunk_sum[j * N + env];
        ga = t.x;
        gp = t.y;
      }
      carry_row_scan(s_a, s_p, tid, g, Ew, Rw, ga, gp);
      C = s_a[e] + s_p[e] * C;
      __syncthreads();
    }
  }

  const long k0 = lo + (long)g * kCarryG;
  double ta[kCarryG], tp[kCarryG];
#pragma unroll
  for (int j = 0; j < kCarryG; ++j) {
    const long k = k0 + j;
    if (ok && k < hi) {
      const double2 t = summary[k * N + env];
      ta[j] = t.x;
      tp[j] = t.y;
    } else {
      ta[j] = 0.0;
      tp[j] = 1.0;
    }
  }
  double ga = 0.0, gp = 1.0;
#pragma unroll
  for (int j = kCarryG - 1; j >= 0; --j) {
    ga = ta[j] + tp[j] * ga;
    gp = prod_nz(tp[j], gp);
  }
  carry_row_scan(s_a, s_p, tid, g, Ew, Rw, ga, gp);
  if constexpr (kCompose) {
    if (g == 0 && ok) chunk_sum[c * N + env] = make_double2(s_a[e], s_p[e]);
  } else {
    double cc = (g + 1 < Rw) ? s_a[tid + Ew] + s_p[tid + Ew] * C : C;
#pragma unroll
    for (int j = kCarryG - 1; j >= 0; --j) {
      const long k = k0 + j;
      if (ok && k < hi) {
        carry[k * N + env] = cc;
        cc = ta[j] + tp[j] * cc;
      }
    }
  }
}

// Strip walk (wide rollouts): one workgroup owns a strip of E adjacent envs
// for the whole horizon and walks it backwards in chunks of S*L steps: a
// thread owns a segment of L steps x VW envs, G = E/VW threads cover a row of
// the strip and S = kStripBlock/G segments make a chunk.  The advantage
// entering a chunk from the right is known when the chunk starts, so one pass
// over the rollout suffices: per chunk each thread forms its segment
// composite (a, P) with a zero carry, a reverse scan composes the segments
// (lane moves inside a wave, then a fold over the waves' composites staged in
// LDS), every thread applies its carry and runs the exact serial recurrence,
// and the chunk's composite applied to the incoming carry is the carry of the
// next chunk to the left.  The next chunk's rows are loaded before the
// current one's arithmetic.  With kStats each block also leaves (n, sum, sum
// of squares) of its fp32 advantages in `partial` for the normaliser.
constexpr int kStripWaves = kStripBlock / kWave;
constexpr int kXcds = 8;

template <int L, int VW>
struct StripRows {
  float r[L][VW], v[L][VW];
  unsigned d[L];  // the row's done bytes as loaded (byte k: env k)
  __device__ __forceinline__ bool done(int i, int k) const {
    if constexpr (VW == 1) return d[i] != 0u;
    else return ((d[i] >> (8 * k)) & 0xffu) != 0u;
  }
};


// Element offsets in the strip walk are 32-bit (rollouts of < 2^30
// elements).  Loads are unconditional (rows past the horizon or the last env
// re-read element 0 and are never used), so a chunk's loads stay in flight
// until its arithmetic needs them.
template <typename T>
__device__ __forceinline__ T* at_byte(T* base, unsigned byte_off) {
  using C = typename std::conditional<std::is_const<T>::value, const char, char>::type;
  return reinterpret_cast<T*>(reinterpret_cast<C*>(base) + byte_off);
}

template <int L, int VW, bool kHasV>
__device__ __forceinline__ void strip_load(const GaeArgs& a, long t0, unsigned e0, bool ok,
                                           StripRows<L, VW>& x) {
  const unsigned n = (unsigned)a.N;
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const unsigned off = (ok && t0 + i < a.T) ? e0 + (unsigned)i * n : 0u;
    load_vec<VW>(at_byte(a.r, off * 4u), x.r[i]);
    if constexpr (kHasV) {
      load_vec<VW>(at_byte(a.v, off * 4u), x.v[i]);
    } else {
#pragma unroll
      for (int k = 0; k < VW; ++k) x.v[i][k] = 0.0f;
    }
    x.d[i] = load_done_raw<VW>(at_byte(a.d, off));
  }
}

// Shared-memory staging of one strip walk (double-buffered by chunk parity).
template <int S, int E>
struct StripShared {
  float v0[2][S][E];                   // first value row of each segment
  double2 wc[2][kStripWaves][E];       // wave composites (a, P) per env
};

// One chunk of the strip walk: rows `x` of chunk c, carry C in and out.
template <int L, int VW, int E, bool kStats>
__device__ __forceinline__ void strip_chunk(const GaeArgs& a, StripShared<kStripBlock / (E / VW), E>& sh,
                                            long c, long env0, bool ok,
                                            const StripRows<L, VW>& cur, const float (&lastv)[VW],
                                            double (&C)[VW],
                                            double (&acc)[3]) {
  constexpr int G = E / VW;           // threads per strip row
  constexpr int S = kStripBlock / G;  // segments per chunk
  constexpr int SW = kWave / G;       // segments per wave
  constexpr long CS = (long)S * L;    // steps per chunk
  const int tid = threadIdx.x;
  const int g = tid % G;
  const int s = tid / G;
  const int w = tid / kWave;
  const int j = (tid % kWave) / G;  // segment index inside the wave
  const unsigned n32 = (unsigned)a.N;
  const int par = (int)(c & 1);
  const long t0 = c * CS + (long)s * L;
  const unsigned e0 = (unsigned)t0 * n32 + (unsigned)env0;
#pragma unroll
  for (int k = 0; k < VW; ++k) sh.v0[par][s][g * VW + k] = cur.v[0][k];
  __syncthreads();
  // value of the step after this segment (the bootstrap past the horizon)
  float nv[VW];
  {
    const bool past = t0 + L >= a.T;
    const int row = s + 1 < S ? s + 1 : 0;
    const int bank = s + 1 < S ? par : par ^ 1;
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      const float x = sh.v0[bank][row][g * VW + k];
      nv[k] = past ? lastv[k] : x;
    }
  }
  const int nvalid = t0 >= a.T ? 0 : (a.T - t0 < L ? (int)(a.T - t0) : L);

  // segment composite with a zero carry, then a reverse inclusive scan over
  // the wave's segments (lane + G*off holds the segment `off` to the right)
  // Each step's delta is formed once (fp64, reference order) and kept for the
  // final pass; gamma*lambda*mask is gl or gl*0, chosen by the done bit.
  const double gl0 = mul(a.gl, 0.0);
  double na[VW], np[VW];
  double dl[L][VW];
#pragma unroll
  for (int k = 0; k < VW; ++k) {
    double ia = 0.0, ip = 1.0;
    double nvd = nv[k];
#pragma unroll
    for (int i = L - 1; i >= 0; --i) {
      if (i < nvalid) {
        const bool done = cur.done(i, k);
        const double vd = (double)cur.v[i][k];
        dl[i][k] = sub(add((double)cur.r[i][k], mul(mul(a.gamma, nvd), done ? 0.0 : 1.0)), vd);
        const double cc = done ? gl0 : a.gl;
        ia = add(dl[i][k], mul(cc, ia));
        ip = mul(ip, cc);
        nvd = vd;
      } else {
        dl[i][k] = 0.0;
      }
    }
#pragma unroll
    for (int off = 1; off < SW; off <<= 1) {
      const double pa = __shfl_down(ia, G * off);
      const double pp = __shfl_down(ip, G * off);
      if (j + off < SW) {
        ia = ia + ip * pa;
        ip = ip * pp;
      }
    }
    na[k] = __shfl_down(ia, G);
    np[k] = __shfl_down(ip, G);
    if (j + 1 >= SW) {
      na[k] = 0.0;
      np[k] = 1.0;
    }
    if (j == 0) sh.wc[par][w][g * VW + k] = make_double2(ia, ip);
  }
  __syncthreads();
  // fold the wave composites from the right: Cw enters this wave, C then
  // enters the chunk to the left
  double Cw[VW];
#pragma unroll
  for (int k = 0; k < VW; ++k) Cw[k] = C[k];
#pragma unroll 4
  for (int ww = kStripWaves - 1; ww >= 0; --ww) {
    if (ww == w) {
#pragma unroll
      for (int k = 0; k < VW; ++k) Cw[k] = C[k];
    }
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      const double2 t = sh.wc[par][ww][g * VW + k];
      C[k] = t.x + t.y * C[k];
    }
  }

  // exact serial recurrence over the segment from its incoming advantage
  float adv[L][VW];
#pragma unroll
  for (int k = 0; k < VW; ++k) {
    double x = na[k] + np[k] * Cw[k];
#pragma unroll
    for (int i = L - 1; i >= 0; --i) {
      if (i < nvalid) {
        const bool done = cur.done(i, k);
        x = add(dl[i][k], mul(done ? gl0 : a.gl, x));
      }
      adv[i][k] = (float)x;
    }
  }
  // this chunk's sums, fp64 (fp32 sums of squares lose the variance when
  // |mean| is large against the spread)
  double s1 = 0.0, s2 = 0.0;
#pragma unroll
  for (int i = 0; i < L; ++i) {
    if (ok && i < nvalid) {
      const unsigned off = (e0 + (unsigned)i * n32) * 4u;
      store_vec<VW>(at_byte(a.adv, off), adv[i]);
      if (a.ret) {
        float rt[VW];
#pragma unroll
        for (int k = 0; k < VW; ++k) rt[k] = adv[i][k] + cur.v[i][k];
        store_vec<VW>(at_byte(a.ret, off), rt);
      }
      if constexpr (kStats) {
#pragma unroll
        for (int k = 0; k < VW; ++k) {
          const double x = (double)adv[i][k];
          s1 += x;
          s2 += x * x;
        }
      }
    }
  }
  if constexpr (kStats) {
    if (ok) {
      acc[0] += (double)(nvalid * VW);
      acc[1] += s1;
      acc[2] += s2;
    }
  }
}

template <int L, int VW, int E, bool kStats, bool kHasV>
__global__ void __launch_bounds__(kStripBlock) gae_strip_kernel(GaeArgs a) {
  constexpr int G = E / VW;           // threads per strip row
  static_assert(E % VW == 0 && kWave % G == 0 && L * VW <= 32, "strip geometry");
  constexpr int S = kStripBlock / G;  // segments per chunk
  constexpr long CS = (long)S * L;    // steps per chunk
  __shared__ StripShared<S, E> sh;

  const int s = threadIdx.x / G;
  // Workgroups are dispatched to the 8 XCDs round-robin; strips are handed
  // out so that each XCD owns a contiguous run of them, and strips that share
  // a 128-byte line of a row share that XCD's L2.
  long strip = blockIdx.x;
  if (gridDim.x % kXcds == 0)
    strip = (long)(blockIdx.x % kXcds) * (gridDim.x / kXcds) + blockIdx.x / kXcds;
  const long env0 = strip * E + (long)(threadIdx.x % G) * VW;
  const bool ok = env0 < a.N;
  const long nch = (a.T + CS - 1) / CS;
  // element offset of this thread's first row in chunk c
  auto row0 = [&](long c) { return (unsigned)((c * CS + (long)s * L) * a.N + env0); };
  auto load = [&](long c, StripRows<L, VW>& x) {
    strip_load<L, VW, kHasV>(a, c * CS + (long)s * L, row0(c), ok && c >= 0, x);
  };

  double C[VW];  // advantage entering the chunk from the right
  float lastv[VW];  // bootstrap value past the horizon
#pragma unroll
  for (int k = 0; k < VW; ++k) {
    C[k] = 0.0;
    lastv[k] = 0.0f;
  }
  if (a.lastv && ok) load_vec<VW>(a.lastv + env0, lastv);
  double acc[3] = {0.0, 0.0, 0.0};

  // The next chunk's rows are in flight while a chunk is processed (two row
  // buffers, the loop unrolled over them).  Every load is unconditional (the
  // chunk before the first one reads element 0 in every lane, one cache
  // line), so the compiler's wait counts stay exact: a load under a branch
  // makes the next join wait for every load in flight.  (Measured: prefetching
  // two chunks ahead is no faster.)
  StripRows<L, VW> b0, b1;
  load(nch - 1, b0);
  for (long c = nch - 1;;) {
    load(c - 1, b1);
    strip_chunk<L, VW, E, kStats>(a, sh, c, env0, ok, b0, lastv, C, acc);
    if (--c < 0) break;
    load(c - 1, b0);
    strip_chunk<L, VW, E, kStats>(a, sh, c, env0, ok, b1, lastv, C, acc);
    if (--c < 0) break;
  }
  if constexpr (kStats) {
    block_sum<3>(acc);
    if (threadIdx.x == 0) {
      a.partial[blockIdx.x * 4 + 0] = acc[0];
      a.partial[blockIdx.x * 4 + 1] = acc[1];
      a.partial[blockIdx.x * 4 + 2] = acc[2];
      a.partial[blockIdx.x * 4 + 3] = 0.0;
    }
  }
}

// ---------------------------------------------------------------------------
// Narrow rollouts: span passes.
// ---------------------------------------------------------------------------
// Aligned rollouts too narrow for the strip walk (N % 4 == 0).  The env
// columns are cut into strips of E envs (SpanPlan) and time into tiles of
// S = 16 * 256/E steps, so a tile is 4096 elements, handled by a 256-thread
// workgroup as 16 consecutive steps of one env per thread (thread = segment
// s, env e).  A tile's rows are contiguous runs of E floats: they are loaded
// with coalesced float4 / 32-bit loads into LDS (one empty row after every
// 16, so the segments of a wave read different banks) and the outputs leave
// the same way.  Each workgroup owns a span of consecutive tiles of one strip
// (about three spans per CU):
//   1. gae_span_sum_kernel walks its span and leaves the span's composite
//      (a, P) per env: the advantage at the span's first step is a + P * x
//      for the advantage x entering it from the right;
//   2. the tile passes' carry scan (gae_carry_kernel) turns the span
//      composites, laid out [spans][N], into the advantage entering each span;
//   3. gae_span_final_kernel walks its span right to left from that carry: per tile the segment composites, a
//      reverse scan (lane shuffles, then the waves' composites), the carry
//      of every segment, and the exact serial recurrence in fp64 with the
//      reference's operation order.  The tile's composite applied to its
//      carry is the carry of the tile to its left.
// Both passes read the rollout; the second read mostly hits the 256 MB
// Infinity Cache, which the first pass's ordinary (temporal) loads filled.
// (Single passes chaining tiles by a decoupled look-back -- fp64 values
// published by agent-scope atomic stores, polled by atomic loads -- measured
// 1.5-2.7x slower than these passes on MI355X: with HBM saturated by the
// streams, each hop of the carry front costs microseconds, and the tiles'
// waits, 11-20 us each in a trace of 4096-element tiles, held their CUs.
// Persistent workgroups prefetching their next tile did not hide it.)
constexpr int kSpanThreads = 256;
constexpr int kSpanL = 16;
constexpr int kSpanWaves = kSpanThreads / kWave;

template <int E>
struct SpanShared {
  static constexpr int SEG = kSpanThreads / E;  // segments per tile
  static constexpr int S = SEG * kSpanL;        // steps per tile
  static constexpr int R = S + S / 16 + 1;      // padded rows + the next-value row
  float r[R * E];                               // rewards, then advantages
  float v[R * E];                               // values, then returns
  uint8_t d[R * E];                             // done bytes
  double2 wc[kSpanWaves][E];                    // wave composites per env
  double x[E];                                  // carry entering the tile
};

// LDS row of tile row t: one empty row after every 16.
__device__ __forceinline__ int span_row(int t) { return t + (t >> 4); }

// One tile's rows in registers (F float4 of rewards and values, F words of
// done bytes per thread) plus the value after the tile.
template <int E>
struct SpanRegs {
  static constexpr int F = SpanShared<E>::S * (E / 4) / kSpanThreads;
  f4 r[F], v[F];
  unsigned d[F];
  float nvt;
};

// Loads of time tile `tile` of the strip at col0 (unconditional: rows past
// the horizon re-read the tile's first row).
template <int E, bool kHasV>
__device__ __forceinline__ void span_load(const GaeArgs& a, long tile, long col0,
                                          SpanRegs<E>& x) {
  constexpr int S = SpanShared<E>::S, G4 = E / 4;
  const long t0 = tile * S;
  const int nrows = (int)std::min<long>(S, a.T - t0);
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < SpanRegs<E>::F; ++k) {
    const int f = tid + k * kSpanThreads;
    const int row = f / G4, q = f % G4;
    const long off = (row < nrows ? t0 + row : t0) * a.N + col0 + q * 4;
    x.r[k] = ld(reinterpret_cast<const f4*>(a.r + off));
    if constexpr (kHasV) x.v[k] = ld(reinterpret_cast<const f4*>(a.v + off));
    x.d[k] = ld(reinterpret_cast<const unsigned*>(a.d + off));
  }
  x.nvt = 0.0f;
  if constexpr (kHasV) {
    const long tn = t0 + S;
    x.nvt = ld(a.v + (tn < a.T ? tn * a.N : 0) + col0 + (tid % E));
  }
}

template <int E, bool kHasV>
__device__ __forceinline__ void span_stage(SpanShared<E>& sh, const SpanRegs<E>& x) {
  constexpr int G4 = E / 4;
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < SpanRegs<E>::F; ++k) {
    const int f = tid + k * kSpanThreads;
    const int p = span_row(f / G4) * E + (f % G4) * 4;
    *reinterpret_cast<f4*>(&sh.r[p]) = x.r[k];
    if constexpr (kHasV) *reinterpret_cast<f4*>(&sh.v[p]) = x.v[k];
    *reinterpret_cast<unsigned*>(&sh.d[p]) = x.d[k];
  }
  if (tid < E) sh.v[(SpanShared<E>::R - 1) * E + tid] = x.nvt;
}

// Segment composite (zero carry) of this thread's 16 steps from the staged
// tile, its deltas and done bits, and the reverse scan inside the wave:
// (na, np) is the composite of the wave's segments to the right of this one;
// lane j == 0 of each env leaves the wave's composite in sh.wc.
template <int E, bool kHasV>
__device__ __forceinline__ void span_segments(const GaeArgs& a, SpanShared<E>& sh, long t0,
                                              int nrows, float lastv, double (&dl)[kSpanL],
                                              unsigned& dm, int& nvalid, double& na,
                                              double& np) {
  constexpr int SW = kWave / E;  // segments per wave
  const int tid = threadIdx.x;
  const int e = tid % E, s = tid / E, w = tid / kWave, j = (tid % kWave) / E;
  const int sr0 = s * kSpanL;
  nvalid = std::max(0, std::min(kSpanL, nrows - sr0));
  const double gl0 = mul(a.gl, 0.0);
  dm = 0u;
  double ia = 0.0, ip = 1.0;
  {
    const int nrow = sr0 + kSpanL;
    double nvd = t0 + nrow >= a.T ? (double)lastv
                                  : (kHasV ? (double)sh.v[span_row(nrow) * E + e] : 0.0);
#pragma unroll
    for (int i = kSpanL - 1; i >= 0; --i) {
      if (i < nvalid) {
        const int p = span_row(sr0 + i) * E + e;
        const double vd = kHasV ? (double)sh.v[p] : 0.0;
        const bool dn = sh.d[p] != 0;
        dl[i] = sub(add((double)sh.r[p], mul(mul(a.gamma, nvd), dn ? 0.0 : 1.0)), vd);
        const double c = dn ? gl0 : a.gl;
        ia = add(dl[i], mul(c, ia));
        ip = mul(ip, c);
        nvd = vd;
        dm |= (unsigned)dn << i;
      } else {
        dl[i] = 0.0;
      }
    }
  }
#pragma unroll
  for (int off = 1; off < SW; off <<= 1) {
    const double pa = __shfl_down(ia, E * off);
    const double pp = __shfl_down(ip, E * off);
    if (j + off < SW) {
      ia = ia + ip * pa;
      ip = ip * pp;
    }
  }
  na = __shfl_down(ia, E);
  np = __shfl_down(ip, E);
  if (j + 1 >= SW) {
    na = 0.0;
    np = 1.0;
  }
  if (j == 0) sh.wc[w][e] = make_double2(ia, ip);
}

// Composite of the whole tile for env e (after the wave composites are staged).
template <int E>
__device__ __forceinline__ double2 span_tile_composite(const SpanShared<E>& sh, int e) {
  double ta = 0.0, tp = 1.0;
#pragma unroll
  for (int ww = kSpanWaves - 1; ww >= 0; --ww) {
    const double2 c = sh.wc[ww][e];
    ta = c.x + c.y * ta;
    tp = c.y * tp;
  }
  return make_double2(ta, tp);
}

// (strip, span) of this workgroup and its tiles [lo, hi).
struct SpanPos {
  long strip, span, lo, hi;
};
__device__ __forceinline__ SpanPos span_pos(const GaeArgs& a) {
  SpanPos p;
  p.strip = blockIdx.x % a.nstrips;
  p.span = blockIdx.x / a.nstrips;
  p.lo = p.span * a.span_tiles;
  p.hi = std::min(p.lo + a.span_tiles, a.Tt);
  return p;
}

template <int E, bool kHasV>
__global__ void __launch_bounds__(kSpanThreads) gae_span_sum_kernel(GaeArgs a) {
  using Sh = SpanShared<E>;
  __shared__ Sh sh;
  const SpanPos sp = span_pos(a);
  const long col0 = sp.strip * E;
  const int tid = threadIdx.x, e = tid % E;
  const float lastv = a.lastv ? a.lastv[col0 + e] : 0.0f;
  double A = 0.0, P = 1.0;  // composite of the tiles walked so far (threads tid < E)
  SpanRegs<E> x;
  span_load<E, kHasV>(a, sp.hi - 1, col0, x);
  for (long tile = sp.hi - 1; tile >= sp.lo; --tile) {
    span_stage<E, kHasV>(sh, x);
    if (tile > sp.lo) span_load<E, kHasV>(a, tile - 1, col0, x);
    __syncthreads();
    const long t0 = tile * Sh::S;
    double dl[kSpanL], na, np;
    unsigned dm;
    int nvalid;
    span_segments<E, kHasV>(a, sh, t0, (int)std::min<long>(Sh::S, a.T - t0), lastv, dl, dm,
                            nvalid, na, np);
    __syncthreads();
    if (tid < E) {
      const double2 t = span_tile_composite<E>(sh, e);
      A = t.x + t.y * A;
      P = prod_nz(t.y, P);
    }
  }
  if (tid < E) a.summary[sp.span * a.N + col0 + e] = make_double2(A, P);
}

template <int E, bool kStats, bool kHasV>
__global__ void __launch_bounds__(kSpanThreads) gae_span_final_kernel(GaeArgs a) {
  using Sh = SpanShared<E>;
  constexpr int S = Sh::S, G4 = E / 4, F = SpanRegs<E>::F;
  __shared__ Sh sh;
  const SpanPos sp = span_pos(a);
  const long col0 = sp.strip * E;
  const int tid = threadIdx.x, e = tid % E, q = tid / E, w = tid / kWave;
  const float lastv = a.lastv ? a.lastv[col0 + e] : 0.0f;
  SpanRegs<E> x;
  span_load<E, kHasV>(a, sp.hi - 1, col0, x);

  // carry entering the span (from the carry scan over the span composites)
  if (tid < E) sh.x[e] = a.carry[sp.span * a.N + col0 + e];

  double s1 = 0.0, s2 = 0.0;  // (fp64: see strip_chunk)
  double cnt = 0.0;
  for (long tile = sp.hi - 1; tile >= sp.lo; --tile) {
    span_stage<E, kHasV>(sh, x);
    if (tile > sp.lo) span_load<E, kHasV>(a, tile - 1, col0, x);
    __syncthreads();
    const long t0 = tile * S;
    const int nrows = (int)std::min<long>(S, a.T - t0);
    double dl[kSpanL], na, np;
    unsigned dm;
    int nvalid;
    span_segments<E, kHasV>(a, sh, t0, nrows, lastv, dl, dm, nvalid, na, np);
    __syncthreads();
    // carry entering this thread's wave, then its segment
    const double X = sh.x[e];
    double C = X;
    for (int ww = kSpanWaves - 1; ww > w; --ww) {
      const double2 c = sh.wc[ww][e];
      C = c.x + c.y * C;
    }
    const double gl0 = mul(a.gl, 0.0);
    double xv = na + np * C;
    const int sr0 = q * kSpanL;
#pragma unroll
    for (int i = kSpanL - 1; i >= 0; --i) {
      if (i < nvalid) {
        xv = add(dl[i], mul((dm >> i) & 1u ? gl0 : a.gl, xv));
        const float av = (float)xv;
        const int p = span_row(sr0 + i) * E + e;
        const float rt = kHasV ? av + sh.v[p] : av;
        sh.r[p] = av;
        sh.v[p] = rt;
        if constexpr (kStats) {
          s1 += (double)av;
          s2 += (double)av * (double)av;
        }
      }
    }
    if constexpr (kStats) cnt += (double)nvalid;
    __syncthreads();
    if (tid < E) {
      const double2 t = span_tile_composite<E>(sh, e);
      sh.x[e] = t.x + t.y * X;  // carry of the tile to the left
    }
#pragma unroll
    for (int k = 0; k < F; ++k) {
      const int f = tid + k * kSpanThreads;
      const int row = f / G4, c4 = f % G4;
      if (row < nrows) {
        const int p = span_row(row) * E + c4 * 4;
        const long off = (t0 + row) * a.N + col0 + c4 * 4;
        st(*reinterpret_cast<const f4*>(&sh.r[p]), reinterpret_cast<f4*>(a.adv + off));
        if (a.ret) st(*reinterpret_cast<const f4*>(&sh.v[p]), reinterpret_cast<f4*>(a.ret + off));
      }
    }
    __syncthreads();
  }
  if constexpr (kStats) {
    double acc[3] = {cnt, s1, s2};
    block_sum<3>(acc);
    if (tid == 0) {
      a.partial[blockIdx.x * 4 + 0] = acc[0];
      a.partial[blockIdx.x * 4 + 1] = acc[1];
      a.partial[blockIdx.x * 4 + 2] = acc[2];
      a.partial[blockIdx.x * 4 + 3] = 0.0;
    }
  }
}

template <int E>
void span_kernels_e(bool norm, bool has_v, const void*& k1, const void*& k2) {
  k1 = has_v ? (const void*)gae_span_sum_kernel<E, true> : (const void*)gae_span_sum_kernel<E, false>;
  if (norm)
    k2 = has_v ? (const void*)gae_span_final_kernel<E, true, true>
               : (const void*)gae_span_final_kernel<E, true, false>;
  else
    k2 = has_v ? (const void*)gae_span_final_kernel<E, false, true>
               : (const void*)gae_span_final_kernel<E, false, false>;
}

void span_kernels(int E, bool norm, bool has_v, const void*& k1, const void*& k2) {
  switch (E) {
    case 64: span_kernels_e<64>(norm, has_v, k1, k2); break;
    case 32: span_kernels_e<32>(norm, has_v, k1, k2); break;
    case 16: span_kernels_e<16>(norm, has_v, k1, k2); break;
    case 8: span_kernels_e<8>(norm, has_v, k1, k2); break;
    default: span_kernels_e<4>(norm, has_v, k1, k2); break;
  }
}

int launch_span(long T, long N, GaeArgs a, bool norm, hipStream_t stream) {
  const void *k1, *k2;
  SpanPlan sp = span_plan(T, N, kSpanMaxBlocks);
  span_kernels(sp.E, norm, a.v != nullptr, k1, k2);
  const long resident = resident_blocks(k2, kSpanThreads, 0, 3 * 256);
  sp = span_plan(T, N, std::min(kSpanMaxBlocks, resident));
  a.nstrips = sp.nstrips;
  a.spans = sp.spans;
  a.span_tiles = sp.tps;
  a.Tt = sp.tt;
  const dim3 grid((unsigned)(sp.nstrips * sp.spans));
  void* args[] = {&a};
  int st;
  if ((st = hip_status(hipLaunchKernel(k1, grid, dim3(kSpanThreads), args, 0, stream)))) return st;
  // carries of the spans: the tile passes' carry scan over [spans][N]
  const CarryPlan cp = make_carry_plan(sp.spans, N);
  const dim3 cgrid((unsigned)cp.groups, (unsigned)cp.nchunks);
  double* carry = const_cast<double*>(a.carry);
  if (cp.nchunks > 1) {
    hipLaunchKernelGGL(gae_carry_kernel<true>, cgrid, dim3(cp.Ew * cp.Rw), 0, stream, a.summary,
                       carry, a.chunk_sum, sp.spans, N, cp.Ew, cp.Rw, cp.nchunks);
    if ((st = last_launch_status())) return st;
  }
  hipLaunchKernelGGL(gae_carry_kernel<false>, cgrid, dim3(cp.Ew * cp.Rw), 0, stream, a.summary,
                     carry, a.chunk_sum, sp.spans, N, cp.Ew, cp.Rw, cp.nchunks);
  if ((st = last_launch_status())) return st;
  if ((st = hip_status(hipLaunchKernel(k2, grid, dim3(kSpanThreads), args, 0, stream)))) return st;
  if (!norm) return PPO_OK;
  return launch_normalize(a.partial, sp.nstrips * sp.spans, a.eps, a.adv, a.adv_n, a.T * a.N,
                          a.hdr, a.stats_out, stream);
}

// ---------------------------------------------------------------------------
// Resident pass: the whole rollout in registers, one launch.
// ---------------------------------------------------------------------------
// Each workgroup (kResBlock threads) owns a tile of E adjacent envs x TS consecutive
// steps (ResPlan); thread (segment s, env-group g) owns 4 envs x L steps.
// All of a tile's loads are issued at once and its rows stay in registers
// until the normalised advantages are stored, so the rollout is read once and
// each output written once (21 bytes per element with the normaliser):
//   1. per thread, the segment composite (a, P) with a zero carry (fp64,
//      reference operation order); a reverse scan over the segments (lane
//      shuffles, then the waves' composites in LDS) gives every segment
//      the composite of the segments to its right and the tile its own.
//   2. a tile publishes its per-env composite; the advantage entering it is
//      the fold of the composites of the tiles to its right in the same env
//      column, read in parallel (one composite per thread) and folded in
//      order from the horizon's end.  Without the normaliser the fold is
//      walked from the nearest tile and stops at a zero factor product (a
//      done flag); a tile skipped that way whose composite is not finite is
//      found after the stores, and the tiles it makes NaN are rewritten.
//   3. with the normaliser, the workgroup publishes (n, sum, sum of squares)
//      of its advantages at once: step 1 also summed each step's suffix
//      composite (a_t, P_t) and their products, and the advantage at step t
//      is a_t + P_t x for the carry x entering the segment, so the sums are
//      closed-form in x (fp64 advantages, fp32 per-thread sums).  Then each
//      thread applies its carry and runs the exact serial recurrence,
//      storing each row of adv and ret as soon as it is done.
//   4. every workgroup reads all partials in the same fixed order, so all
//      derive bit-identical mean and std (the partials were published before
//      step 3, so the wait overlaps it), and stores the normalised
//      advantages from the registers.
// Cross-workgroup values travel through the self-validating slots of
// grid_sync.hpp (start barrier, bounded waits); the host launches the pass
// only when the whole grid fits on the device at once, so every producer
// runs while its consumers wait.
constexpr int kResWaves = kResBlock / kWave;
#ifdef PPO_GAE_RES_TRACE
// Phase timestamps of the resident pass (wall clock, 100 MHz), one row of
// kResTraceRow words per workgroup (6 marks per round): a measurement build
// only.
constexpr int kResTraceRow = 64;
static_assert(6 * kResMaxRounds <= kResTraceRow, "a trace row holds every round's marks");
__device__ uint64_t g_res_trace[4096 * kResTraceRow];
#define RES_MARK(k)                                                                   \
  if (threadIdx.x == 0)                                                               \
  g_res_trace[blockIdx.x * kResTraceRow + (k) + 6 * res_round] = wall_clock64()
#else
#define RES_MARK(k)
#endif

template <int E>
struct ResShared {
  static constexpr int Q = kResBlock / E;   // look-back chunks per env
  double2 wc[kResWaves][E];                 // wave composites (a, P) per env
  double2 lb[Q][E];                         // look-back: composite of each chunk of tiles
  float ssum[5][4][kResBlock];              // per thread and env: sums of a, P, aa, aP, PP
  double carry[E];                          // advantage entering the tile
  float norm[2];                            // mean and denominator
  double mean, m2;                          // the statistics' fp64 mean and centred sum of squares
  int exact;                                // the second, exact pass is run
  int rest;                                 // the look-back's full fold is needed
  int bad;                                  // a composite of this workgroup's tiles is not finite
  int nanfl[E];                             // the exact carry entering the tile is NaN
};

template <int E, int L, bool kStats, bool kHasV, bool kRounds>
__global__ void __launch_bounds__(kResBlock) gae_resident_kernel(GaeArgs a) {
  constexpr int VW = 4;
  constexpr int G = E / VW;            // threads per tile row
  constexpr int SW = kWave / G;        // segments per wave
  constexpr int S = kResBlock / G;     // segments per tile
  constexpr long TS = (long)S * L;     // steps per tile
  constexpr int Q = ResShared<E>::Q;
  constexpr int LB = 4;                // look-back tiles in flight per thread
  static_assert(kWave % G == 0 && L <= 32, "resident geometry");
  static_assert(!(kStats && kRounds), "the normaliser needs every advantage resident at once");
  __shared__ ResShared<E> sh;

  const int tid = threadIdx.x;
  const int g = tid % G, sg = tid / G, w = tid / kWave, j = (tid % kWave) / G;
  // (kRounds = false: one round, the whole horizon)
  const long nc = a.res_nc, nt = a.res_nt;
  const long ntr = kRounds ? a.res_ntr : nt, rounds = kRounds ? a.res_rounds : 1;
  // workgroup b owns, in each round, time tile `tl` of the round (0 = the
  // round's last steps) of env column `col`; rounds run from the end of the
  // horizon backwards, and the first workgroups take the tiles whose
  // composites the others wait for
  const long col = (long)blockIdx.x % nc, tl = (long)blockIdx.x / nc;
  const long env0 = col * E + (long)g * VW;
  const unsigned n32 = (unsigned)a.N;
  uint64_t* ctr = a.slots;
  uint64_t* comp = a.slots + kResSlotBase;           // [nt][nc][E][2]
  uint64_t* bnd = comp + (size_t)nt * nc * 2 * E;    // [rounds][N]
  uint64_t* part = bnd + (size_t)rounds * a.N;       // [grid][kResPartWords]
  auto tile_tt = [&](long rd) { return nt - 1 - (rd * ntr + tl); };  // < 0: no tile
  int fail = 0;  // one of this thread's bounded waits gave up
  // The composite of chunk q (of Q) of tiles lo + 1 .. hi for env e, folded
  // from the right, LB slot pairs in flight; `base`/`step` address the slot
  // pair of tile u for env e: word offset ((u * nc + col) * E + e) * 2.
  auto fold_chunk = [&](int lo, int hi, int q, unsigned base, unsigned step) {
    const int m = hi - lo;               // tiles to fold
    const int cs = (m + Q - 1) / Q;      // tiles per chunk
    const int u_hi = hi - q * cs, u_lo = max(lo + 1, hi - (q + 1) * cs + 1);
    double A = 0.0, P = 1.0;
    for (int u0 = u_hi; u0 >= u_lo; u0 -= LB) {
      uint64_t wa[LB], wp[LB];
#pragma unroll
      for (int k = 0; k < LB; ++k) {
        wa[k] = wp[k] = 0;
        if (u0 - k >= u_lo) {
          uint64_t* sl = comp + (base + (unsigned)(u0 - k) * step);
          wa[k] = slot_peek(sl);
          wp[k] = slot_peek(sl + 1);
        }
      }
#pragma unroll
      for (int k = 0; k < LB; ++k) {
        if (u0 - k >= u_lo) {
          uint64_t* sl = comp + (base + (unsigned)(u0 - k) * step);
          const double ca = slot_or_get(wa[k], sl, a.wc.spin, fail);
          const double cp = slot_or_get(wp[k], sl + 1, a.wc.spin, fail);
          A = ca + cp * A;
          P = prod_nz(cp, P);
        }
      }
    }
    return make_double2(A, P);
  };
  // (without the normaliser) this workgroup's flag of non-finite composites,
  // published once its last tile's composite is
  auto publish_bad = [&]() {
    if (!kStats && tid == 0)
      slot_put(part + (size_t)blockIdx.x * kResPartWords, sh.bad ? 1.0 : 0.0);
  };
#ifdef PPO_GAE_RES_TRACE
  long res_round = 0;
#endif
  RES_MARK(0);
  // Wave 0 empties the slots this workgroup will fill (its tiles' composites,
  // a round's left-edge carries, its partial), waits until those stores are
  // done, and arrives at the start barrier; no workgroup reads a slot before
  // the barrier is complete, so no reader can see what the slot held before
  // this call.  The other waves start their loads meanwhile.
  // this launch's barrier tag and the call counter it came from, kept in
  // LDS by thread 0 (its only user) rather than in registers across step 1
  __shared__ unsigned s_tag;
  __shared__ uint64_t s_epoch;
  if (tid == 0) sh.bad = 0;
  if (w == 0) {
    for (long rd = 0; rd < rounds; ++rd) {
      const long tt = tile_tt(rd);
      if (tt > 0) {
        for (int q = tid; q < 2 * E; q += kWave)
          slot_clear(comp + (size_t)(tt * nc + col) * 2 * E + q);
        if (tl == ntr - 1 && rd + 1 < rounds && tid < E)
          slot_clear(bnd + (size_t)rd * a.N + col * E + tid);
      }
    }
    uint64_t epoch;
    const unsigned tag = launch_tag(&a.hdr->epoch, a.nonce, epoch);
    if (tid == 0) {
      s_tag = tag;
      s_epoch = epoch;
    }
    sync_start(ctr, part + (size_t)blockIdx.x * kResPartWords, (int)kResPartWords, tag);
  }

  const double gl0 = mul(a.gl, 0.0);
  float r[L][VW], v[L][VW], nv[VW];
  unsigned d[L];
  // ---- loads: every row of a segment, unconditional (rows past the
  // horizon re-read row 0), plus the value row after the segment
  auto load_row = [&](long ts0, int i) {
    const unsigned off = (ts0 + i < a.T ? (unsigned)(ts0 + i) * n32 : 0u) + (unsigned)env0;
    load_vec<VW>(at_byte(a.r, off * 4u), r[i]);
    if constexpr (kHasV) {
      load_vec<VW>(at_byte(a.v, off * 4u), v[i]);
    } else {
#pragma unroll
      for (int k = 0; k < VW; ++k) v[i][k] = 0.0f;
    }
    d[i] = load_done_raw<VW>(at_byte(a.d, off));
  };
  // (branch-free: one load from a valid address, zeros selected after; a
  // load under a branch leaves the compiler unable to count the wave's
  // outstanding loads, and it then waits for all of them)
  auto load_next_value = [&](long ts0) {
    const long tn = ts0 + L;
    const bool inner = tn < a.T;
    const float* src = inner ? (kHasV ? a.v + (unsigned)tn * n32 + (unsigned)env0 : a.r + env0)
                             : (a.lastv ? a.lastv + env0 : a.r + env0);
    float x[VW];
    load_vec<VW>(src, x);
    const bool use = inner ? kHasV : a.lastv != nullptr;
#pragma unroll
    for (int k = 0; k < VW; ++k) nv[k] = use ? x[k] : 0.0f;
  };
  int nvalid = 0;
  long t0 = 0;
  // the first round's rows, last row first, as step 1 consumes them; later
  // rounds' rows are loaded row by row as the round before stores its own
  // (software pipelining across rounds: the registers are the buffers).  The
  // value row after the segment goes first: step 1 needs it before any row,
  // and a wave's loads complete in order, so a wait for the last-issued load
  // would be a wait for all of them.
  if (tile_tt(0) >= 0) {
    const long ts0 = tile_tt(0) * TS + (long)sg * L;
    load_next_value(ts0);
#pragma unroll
    for (int i = L - 1; i >= 0; --i) load_row(ts0, i);
  }
  for (long rd = 0; rd < rounds; ++rd) {
    const long tt = tile_tt(rd);
    if (tt < 0) break;  // (the last round may hold fewer tiles)
    t0 = tt * TS + (long)sg * L;
    nvalid = t0 >= a.T ? 0 : (a.T - t0 < L ? (int)(a.T - t0) : L);
    const long tt_next = kRounds && rd + 1 < rounds ? tile_tt(rd + 1) : -1;
#ifdef PPO_GAE_RES_TRACE
    res_round = rd;
#endif
    const long t0_next = tt_next * TS + (long)sg * L;

    // ---- 1. segment composites and the reverse scan inside the tile.  With
    // the normaliser, also the sums over the segment's steps of the suffix
    // composites (a_t, P_t) (steps t..segment end, zero carry) and of their
    // products: the advantage at step t is a_t + P_t x for the carry x
    // entering the segment, so once x is known the segment's sum of
    // advantages and of their squares follow without the advantages.
    double na[VW], np[VW];
    {
      float sa[VW], sp[VW], saa[VW], sap[VW], spp[VW];
      double ia[VW], ip[VW], nvd[VW];
#pragma unroll
      for (int k = 0; k < VW; ++k) {
        ia[k] = 0.0;
        ip[k] = 1.0;
        nvd[k] = nv[k];
        sa[k] = sp[k] = saa[k] = sap[k] = spp[k] = 0.0f;
      }
#pragma unroll
      for (int i = L - 1; i >= 0; --i) {
        if (i < nvalid) {
#pragma unroll
          for (int k = 0; k < VW; ++k) {
            // (the composites only carry the advantage between segments: fp64
            // with fused multiply-adds, 5 operations; the advantages
            // themselves come from the exact recurrence below)
            const bool done = ((d[i] >> (8 * k)) & 0xffu) != 0u;
            const double vd = (double)v[i][k];
            const double dl =
                __builtin_fma(a.gamma * nvd[k], done ? 0.0 : 1.0, (double)r[i][k]) - vd;
            const double cc = done ? gl0 : a.gl;
            ia[k] = __builtin_fma(cc, ia[k], dl);
            ip[k] = ip[k] * cc;
            nvd[k] = vd;
            if constexpr (kStats) {
              const float fa = (float)ia[k], fp = (float)ip[k];
              sa[k] += fa;
              sp[k] += fp;
              saa[k] += fa * fa;
              sap[k] += fa * fp;
              spp[k] += fp * fp;
            }
          }
        }
      }
#pragma unroll
      for (int k = 0; k < VW; ++k) {
        na[k] = ia[k];
        np[k] = ip[k];
        if constexpr (kStats) {
          // parked in LDS until the carries are known (registers are short)
          sh.ssum[0][k][tid] = sa[k];
          sh.ssum[1][k][tid] = sp[k];
          sh.ssum[2][k][tid] = saa[k];
          sh.ssum[3][k][tid] = sap[k];
          sh.ssum[4][k][tid] = spp[k];
        }
      }
    }
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      double ia = na[k], ip = np[k];
#pragma unroll
      for (int off = 1; off < SW; off <<= 1) {
        const double pa = __shfl_down(ia, G * off);
        const double pp = __shfl_down(ip, G * off);
        if (j + off < SW) {
          ia = ia + ip * pa;
          ip = ip * pp;
        }
      }
      na[k] = __shfl_down(ia, G);
      np[k] = __shfl_down(ip, G);
      if (j + 1 >= SW) {
        na[k] = 0.0;
        np[k] = 1.0;
      }
      if (j == 0) sh.wc[w][g * VW + k] = make_double2(ia, ip);
    }
    __syncthreads();
    RES_MARK(1);

    // ---- 2. publish the tile composite
    if (tid < E && tt > 0) {
      double ta = 0.0, tp = 1.0;
#pragma unroll
      for (int ww = kResWaves - 1; ww >= 0; --ww) {
        const double2 c = sh.wc[ww][tid];
        ta = c.x + c.y * ta;
        tp = c.y * tp;
      }
      slot_put(comp + ((size_t)(tt * nc + col) * E + tid) * 2 + 0, ta);
      slot_put(comp + ((size_t)(tt * nc + col) * E + tid) * 2 + 1, tp);
      if (!kStats && !(__builtin_isfinite(ta) && __builtin_isfinite(tp))) sh.bad = 1;
    }
    // the start barrier (once): every workgroup's slots are empty by now
    if (rd == 0 && tid == 0) {
      if (!res_wait(ctr, s_tag, gridDim.x, a.wc.spin)) fail = 1;
      if (blockIdx.x == 0) epoch_advance(&a.hdr->epoch, s_epoch);
    }
    __syncthreads();

    // ---- look-back: the tiles to the right inside this round (hi down to
    // tt + 1), in Q chunks per env, each folded by one thread with its loads
    // in flight together; then the chunks in order, from the carry entering
    // the round (the previous round's left-edge carry, zero for the first)
    {
      // (tile indices fit in 32 bits: at most 256 tiles per round and
      // kResMaxRounds rounds)
      const int e = tid % E, q = tid / E;
      const int hi = (int)(nt - 1 - rd * ntr);
      // slot pair of tile u for env e: word offset ((u * nc + col) * E + e) * 2
      const unsigned step = (unsigned)(nc * E * 2), base = (unsigned)((col * E + e) * 2);
      // Without the normaliser, the carry is first walked from the nearest
      // tile outwards, and the walk stops at a tile whose factor product is
      // zero (a done flag in that env): the tiles beyond it are multiplied by
      // zero.  The window's words are read at once, one tile per thread.
      double S = 0.0, M = 1.0;  // (threads tid < E) carry = S + M x (the rest)
      int lo = (int)tt;         // the full fold covers tiles lo + 1 .. hi
      if constexpr (!kStats) {
        {
          const int u = (int)tt + 1 + q;
          uint64_t wa = 0, wp = 0;
          if (u <= hi) {
            uint64_t* sl = comp + (base + (unsigned)u * step);
            wa = slot_peek(sl);
            wp = slot_peek(sl + 1);
          }
          sh.lb[q][e] = make_double2(__builtin_bit_cast(double, wa), __builtin_bit_cast(double, wp));
          if (tid == 0) sh.rest = 0;
        }
        __syncthreads();
        if (tid < E) {
          int u = (int)tt + 1;
          for (int qq = 0; qq < Q && u <= hi && M != 0.0; ++qq, ++u) {
            const double2 c = sh.lb[qq][e];
            uint64_t* sl = comp + (base + (unsigned)u * step);
            const double ca = slot_or_get(__builtin_bit_cast(uint64_t, c.x), sl, a.wc.spin, fail);
            const double cp =
                slot_or_get(__builtin_bit_cast(uint64_t, c.y), sl + 1, a.wc.spin, fail);
            S = S + M * ca;
            M = prod_nz(M, cp);
          }
          if (M != 0.0 && u <= hi) sh.rest = 1;
        }
        __syncthreads();
        lo = (int)tt + Q;
      }
      if (kStats || sh.rest) {
        // (the window's words in sh.lb were read before the last barrier)
        sh.lb[q][e] = fold_chunk(lo, hi, q, base, step);
        __syncthreads();
      }
      if (tid < E) {
        double xc = 0.0;
        if (kStats || sh.rest || M != 0.0) {
          xc = rd > 0 ? slot_get(bnd + (size_t)(rd - 1) * a.N + col * E + e, a.wc.spin, fail)
                      : 0.0;
          if (kStats || sh.rest)
            for (int qq = 0; qq < Q; ++qq) {
              const double2 c = sh.lb[qq][e];
              xc = c.x + c.y * xc;
            }
        }
        sh.carry[e] = kStats ? xc : S + M * xc;
      }
      __syncthreads();
    }
    RES_MARK(2);
    if (rd == rounds - 1) publish_bad();

    // ---- 3. carry entering each of this thread's segments (one per env)
    double x[VW];
#pragma unroll
    for (int k = 0; k < VW; ++k) {
      const int e = g * VW + k;
      double C = sh.carry[e];
      for (int ww = kResWaves - 1; ww > w; --ww) {
        const double2 c = sh.wc[ww][e];
        C = c.x + c.y * C;
      }
      x[k] = na[k] + np[k] * C;
    }
    // a round's left-edge tile hands the advantage at its left edge to the
    // next round
    if (tl == ntr - 1 && rd + 1 < rounds && tt > 0 && tid < E) {
      double C = sh.carry[tid];
#pragma unroll
      for (int ww = kResWaves - 1; ww >= 0; --ww) {
        const double2 c = sh.wc[ww][tid];
        C = c.x + c.y * C;
      }
      slot_put(bnd + (size_t)rd * a.N + col * E + tid, C);
    }
    if constexpr (kStats) {
      // the statistics partial (a single round), published before this
      // workgroup's stores
      double acc[3] = {(double)(nvalid * VW), 0.0, 0.0};
#pragma unroll
      for (int k = 0; k < VW; ++k) {
        const double sa = sh.ssum[0][k][tid], sp = sh.ssum[1][k][tid];
        const double saa = sh.ssum[2][k][tid], sap = sh.ssum[3][k][tid], spp = sh.ssum[4][k][tid];
        acc[1] += sa + sp * x[k];
        acc[2] += saa + 2.0 * sap * x[k] + spp * x[k] * x[k];
      }
      block_sum_lds<3>(acc);
      if (tid == 0) {
        uint64_t* pp = part + (size_t)blockIdx.x * kResPartWords;
        slot_put(pp + 0, acc[0]);
        slot_put(pp + 1, acc[1]);
        slot_put(pp + 2, acc[2]);
      }
    }

    // ---- exact recurrence from each segment's carry, adv and ret.  The
    // deltas are formed again from the rows rather than kept from step 1
    // (fp64, two registers each): the empty asm hides from the compiler that
    // the rows are unchanged, so it cannot keep step 1's values alive instead.
#pragma unroll
    for (int i = 0; i < L; ++i) {
#pragma unroll
      for (int k = 0; k < VW; ++k) asm volatile("" : "+v"(r[i][k]), "+v"(v[i][k]));
    }
#pragma unroll
    for (int i = 0; i < L; ++i) asm volatile("" : "+v"(d[i]));
    {
      double nvd[VW];
#pragma unroll
      for (int k = 0; k < VW; ++k) nvd[k] = nv[k];
      if constexpr (kRounds) {
        // (first of the next round's loads; after the last round, rows past
        // the horizon: every thread re-reads row 0, unconditionally)
        load_next_value(tt_next >= 0 ? t0_next : a.T);
      }
      // rows from the last: each row is stored as soon as its 4 envs are done
#pragma unroll
      for (int i = L - 1; i >= 0; --i) {
        if (i < nvalid) {
#pragma unroll
          for (int k = 0; k < VW; ++k) {
            const bool done = ((d[i] >> (8 * k)) & 0xffu) != 0u;
            const double vd = (double)v[i][k];
            const double dl =
                sub(add((double)r[i][k], mul(mul(a.gamma, nvd[k]), done ? 0.0 : 1.0)), vd);
            x[k] = add(dl, mul(done ? gl0 : a.gl, x[k]));
            nvd[k] = vd;
            r[i][k] = (float)x[k];  // the advantage replaces the reward
          }
          const unsigned off = ((unsigned)(t0 + i) * n32 + (unsigned)env0) * 4u;
          // With the normaliser, the raw advantages are the output a PPO step
          // does not read next (the loss reads the normalised advantages and
          // the returns, which stay temporal and are then read from the
          // Infinity Cache): written nontemporally where the tile's rows are
          // whole lines, they leave no dirty lines to be written back during
          // the next kernel.  Measured on MI355X, T x N = 2048 x 4096: PPO step
          // 294.4 -> 292.4 us, back-to-back calls 46.8 -> 40.7 us.
          // Normalised in place (adv_n aliases adv), the raw advantages are
          // overwritten below from these registers: not stored at all.
          if constexpr (kStats && E >= 32) {
            if (a.adv != a.adv_n) store_vec_nt<VW>(at_byte(a.adv, off), r[i]);
          } else if (!kStats || a.adv != a.adv_n) {
            store_vec<VW>(at_byte(a.adv, off), r[i]);
          }
          if (a.ret) {
            float rt[VW];
#pragma unroll
            for (int k = 0; k < VW; ++k) rt[k] = r[i][k] + v[i][k];
            store_vec<VW>(at_byte(a.ret, off), rt);
          }
        }
        if constexpr (kRounds) load_row(tt_next >= 0 ? t0_next : a.T, i);  // next round's row i
      }
    }
    RES_MARK(3);
    if constexpr (kStats) {
      // ---- 4. statistics of all advantages (every workgroup reads all partials
      // in the same fixed order, so all derive bit-identical mean and std), then
      // the normalised advantages from the registers
      {
        double tot[3] = {0.0, 0.0, 0.0};
        for (long u = tid; u < (long)gridDim.x; u += kResBlock) {
          uint64_t* pp = part + (size_t)u * kResPartWords;
          tot[0] += slot_get(pp + 0, a.wc.spin, fail);
          tot[1] += slot_get(pp + 1, a.wc.spin, fail);
          tot[2] += slot_get(pp + 2, a.wc.spin, fail);
        }
        block_sum_lds<3>(tot);
        if (tid == 0) {
          const double mean = tot[1] / tot[0];
          const double m2 = tot[2] - tot[1] * mean;
          sh.mean = mean;
          sh.m2 = m2;
          // The workgroups' sums come from fp32 closed forms, whose rounding
          // (relative ~1e-7 of the sum of squares) swamps the variance once
          // |mean| is large against the spread.  Past mean^2 > 100 var the
          // centred sum of squares is therefore formed exactly, in a second
          // exchange over the advantages held in registers.  Every workgroup
          // has the same totals, so all take the same branch.
          sh.exact = tot[0] > 1.0 && mean * mean * tot[0] > 100.0 * (m2 > 0.0 ? m2 : 0.0);
        }
        lds_barrier();
        if (sh.exact) {
          const double mean = sh.mean;
          double c[1] = {0.0};
#pragma unroll
          for (int i = 0; i < L; ++i) {
            if (i < nvalid) {
#pragma unroll
              for (int k = 0; k < VW; ++k) {
                const double dx = (double)r[i][k] - mean;
                c[0] += dx * dx;
              }
            }
          }
          block_sum_lds<1>(c);
          if (tid == 0) slot_put(part + (size_t)blockIdx.x * kResPartWords + 3, c[0]);
          double t2[1] = {0.0};
          for (long u = tid; u < (long)gridDim.x; u += kResBlock)
            t2[0] += slot_get(part + (size_t)u * kResPartWords + 3, a.wc.spin, fail);
          block_sum_lds<1>(t2);
          if (tid == 0) sh.m2 = t2[0];
        }
        if (tid == 0) {
          // norm_params' formulas on these totals
          const double n = tot[0];
          const double mean = sh.mean, m2 = sh.m2;
          float mean_f = (float)mean, std_f, mean_used, denom;
          if (n > 1.0) {
            std_f = (float)sqrt((m2 > 0.0 ? m2 : 0.0) / (n - 1.0));
            mean_used = mean_f;
            denom = std_f + (float)a.eps;
          } else {
            std_f = __builtin_nanf("");
            mean_used = 0.0f;
            denom = 1.0f;
          }
          sh.norm[0] = mean_used;
          sh.norm[1] = denom;
          if (blockIdx.x == 0) {
            a.hdr->stats[0] = mean_used;
            a.hdr->stats[1] = std_f;
            a.hdr->stats[2] = denom;
            if (a.stats_out) {
              a.stats_out[0] = mean_f;
              a.stats_out[1] = std_f;
            }
          }
        }
        lds_barrier();
      }
      RES_MARK(4);
      const float mean = sh.norm[0], denom = sh.norm[1];
#pragma unroll
      for (int i = 0; i < L; ++i) {
        if (i < nvalid) {
          const unsigned off = ((unsigned)(t0 + i) * n32 + (unsigned)env0) * 4u;
          float y[VW];
#pragma unroll
          for (int k = 0; k < VW; ++k) y[k] = (r[i][k] - mean) / denom;
          store_vec<VW>(at_byte(a.adv_n, off), y);
        }
      }
      RES_MARK(5);
    }
    lds_barrier();  // this round's LDS (composites, carries) is read before the next overwrites it
  }
  // (a workgroup without a tile in the last round publishes its flag here)
  if (tile_tt(rounds - 1) < 0) publish_bad();
  if constexpr (!kStats) {
    // The look-back's walk stops at a zero factor product and skips the tiles
    // beyond it, which is exact unless a skipped composite is not finite: the
    // reference then carries 0 x inf (or 0 x NaN) = NaN into the tile, and
    // every advantage and return of that env in the tile is NaN.  Once every
    // workgroup has published whether its composites are all finite (they
    // publish before their own look-back), a workgroup that sees any that are
    // not folds every composite to the right of each of its tiles (all
    // rounds, in chunks) and writes NaN over the envs whose carry is NaN.  The
    // same threads wrote those elements, so the NaN is the value that stays.
    int any = 0;
    for (long u = tid; u < (long)gridDim.x; u += kResBlock)
      any |= !(slot_get(part + (size_t)u * kResPartWords, a.wc.spin, fail) == 0.0);
    if (__syncthreads_or(any)) {
      const int e = tid % E, q = tid / E;
      const unsigned step = (unsigned)(nc * E * 2), base = (unsigned)((col * E + e) * 2);
      for (long rd = 0; rd < rounds; ++rd) {
        const long tt = tile_tt(rd);
        if (tt < 0) break;
        sh.lb[q][e] = fold_chunk((int)tt, (int)nt - 1, q, base, step);
        __syncthreads();
        if (tid < E) {
          double xc = 0.0;
          for (int qq = 0; qq < Q; ++qq) {
            const double2 c = sh.lb[qq][e];
            xc = c.x + c.y * xc;
          }
          sh.nanfl[e] = xc != xc;
        }
        __syncthreads();
        const long t0r = tt * TS + (long)sg * L;
        const int nvr = t0r >= a.T ? 0 : (a.T - t0r < L ? (int)(a.T - t0r) : L);
        const float qnan = __builtin_nanf("");
        for (int k = 0; k < VW; ++k) {
          if (!sh.nanfl[g * VW + k]) continue;
          for (int i = 0; i < nvr; ++i) {
            const unsigned off = ((unsigned)(t0r + i) * n32 + (unsigned)(env0 + k)) * 4u;
            *(float*)at_byte(a.adv, off) = qnan;
            if (a.ret) *(float*)at_byte(a.ret, off) = qnan;
          }
        }
        __syncthreads();
      }
    }
  }
  // A wait that gave up (grid not co-resident) may have read slots another
  // workgroup had not yet emptied or filled: this workgroup writes NaN over
  // every output element it wrote (its own threads' elements, so the NaN is
  // the value that stays) and raises the device's wait-status word.
  if (__syncthreads_or(fail)) {
    if (tid == 0) wait_report(a.wc.status);
    const float qnan = __builtin_nanf("");
    for (long rd = 0; rd < rounds; ++rd) {
      const long tt = tile_tt(rd);
      if (tt < 0) break;
      const long t0r = tt * TS + (long)sg * L;
      const int nvr = t0r >= a.T ? 0 : (a.T - t0r < L ? (int)(a.T - t0r) : L);
      for (int i = 0; i < nvr; ++i)
        for (int k = 0; k < VW; ++k) {
          const unsigned off = ((unsigned)(t0r + i) * n32 + (unsigned)(env0 + k)) * 4u;
          *(float*)at_byte(a.adv, off) = qnan;
          if (a.ret) *(float*)at_byte(a.ret, off) = qnan;
          if constexpr (kStats) *(float*)at_byte(a.adv_n, off) = qnan;
        }
    }
  }
}

template <int E, int L>
const void* res_kernel_el(bool stats, bool has_v) {
  if (stats)
    return has_v ? (const void*)gae_resident_kernel<E, L, true, true, false>
                 : (const void*)gae_resident_kernel<E, L, true, false, false>;
  return has_v ? (const void*)gae_resident_kernel<E, L, false, true, false>
               : (const void*)gae_resident_kernel<E, L, false, false, false>;
}

template <int E>
const void* res_kernel_e(int L, bool stats, bool has_v, bool rounds) {
  if (rounds)  // (rounds always use 16 steps per thread and no normaliser)
    return has_v ? (const void*)gae_resident_kernel<E, 16, false, true, true>
                 : (const void*)gae_resident_kernel<E, 16, false, false, true>;
  return L == 16 ? res_kernel_el<E, 16>(stats, has_v)
                 : (L == 8 ? res_kernel_el<E, 8>(stats, has_v) : res_kernel_el<E, 4>(stats, has_v));
}

const void* res_kernel(const ResPlan& rp, bool stats, bool has_v) {
  const bool rounds = rp.rounds > 1;
  if (rp.E == 128 && !rounds) return res_kernel_el<128, 16>(stats, has_v);
  if (rp.E == 128) return nullptr;  // (not planned: rounds use at most 64-env tiles)
  if (rp.E == 64) return res_kernel_e<64>(rp.L, stats, has_v, rounds);
  if (rp.E == 32) return res_kernel_e<32>(rp.L, stats, has_v, rounds);
  return res_kernel_e<16>(rp.L, stats, has_v, rounds);
}

// The environment variable PPO_AMD_GAE_RESIDENT=0 turns the resident pass
// off (every rollout then takes the strip walk, span or tile passes), so that
// those paths can be tested on shapes the resident pass would take.
bool resident_ok(long T, long N, bool norm, bool has_v) {
  const char* env = getenv("PPO_AMD_GAE_RESIDENT");
  if (env && env[0] == '0') return false;
  const ResPlan rp = res_plan(T, N, norm);
  if (rp.E == 0) return false;
  const void* kern = res_kernel(rp, norm, has_v);
  return kern && resident_blocks(kern, kResBlock, 0, 0) >= rp.grid();
}

// Launches the resident pass when the plan applies and the whole grid fits
// on the device at once; returns -1 (nothing launched) otherwise.
int launch_resident(long T, long N, GaeArgs a, bool norm, hipStream_t stream) {
  if (!resident_ok(T, N, norm, a.v != nullptr)) return -1;
  const ResPlan rp = res_plan(T, N, norm);
  const void* kern = res_kernel(rp, norm, a.v != nullptr);
  a.res_nc = rp.nc;
  a.res_nt = rp.nt;
  a.res_ntr = rp.ntr;
  a.res_rounds = rp.rounds;
  a.nonce = next_nonce();
  int st = wait_ctl(a.wc);
  if (st) return st;
  void* args[] = {&a};
  return hip_status(
      hipLaunchKernel(kern, dim3((unsigned)rp.grid()), dim3(kResBlock), args, 0, stream));
}

// Pass kernels by (VW, L, solo) geometry.
template <int kMode>
const void* tile_kernel(int vw, const PassGeom& g) {
  if (vw == 1) return (const void*)gae_tile_kernel<1, 16, kStacked, kMode>;
  if (g.solo) return (const void*)gae_tile_kernel<4, 16, kSoloTile, kMode>;
  return (const void*)gae_tile_kernel<4, 4, kStacked, kMode>;
}

// Strip-walk kernel for strips of E envs.
template <int E>
const void* strip_kernel_e(bool norm, bool has_v) {
  if (norm)
    return has_v ? (const void*)gae_strip_kernel<kStripL, 1, E, true, true>
                 : (const void*)gae_strip_kernel<kStripL, 1, E, true, false>;
  return has_v ? (const void*)gae_strip_kernel<kStripL, 1, E, false, true>
               : (const void*)gae_strip_kernel<kStripL, 1, E, false, false>;
}

const void* strip_kernel(int E, bool norm, bool has_v) {
  if (E == 32) return strip_kernel_e<32>(norm, has_v);
  if (E == 16) return strip_kernel_e<16>(norm, has_v);
  return strip_kernel_e<8>(norm, has_v);
}

int launch_tile(const void* kern, const PassGeom& g, GaeArgs a, long Tt, hipStream_t stream) {
  a.Tq = g.Tq;
  a.Qw = g.Qw;
  a.Sw = g.Sw;
  void* args[] = {&a};
  return hip_status(hipLaunchKernel(kern, dim3((unsigned)(Tt * g.Tq)), dim3(kBlock), args, 0,
                                    stream));
}

int launch_gae(const GaePlan& p, GaeArgs a, bool norm, hipStream_t stream) {
  a.Q = p.Q;
  a.Tt = p.Tt;
  a.span = p.span;
  int st;
  const StripPlan sp = strip_plan(p);
  if (sp.E > 0) {
    void* args[] = {&a};
    const void* kern = strip_kernel(sp.E, norm, a.v != nullptr);
    if ((st = hip_status(hipLaunchKernel(kern, dim3((unsigned)sp.strips), dim3(kStripBlock), args,
                                         0, stream))))
      return st;
    if (!norm) return PPO_OK;
    return launch_normalize(a.partial, sp.strips, a.eps, a.adv, a.adv_n, a.T * a.N, a.hdr,
                            a.stats_out, stream);
  }
  if (p.Tt > 1) {
    // pass 1: tile composites; then the carry scan
    const PassGeom& g1 = p.scan;
    if ((st = launch_tile(tile_kernel<kSummary>(p.vw, g1), g1, a, p.Tt, stream))) return st;
    const CarryPlan cp = make_carry_plan(p.Tt, a.N);
    const dim3 cgrid((unsigned)cp.groups, (unsigned)cp.nchunks);
    if (cp.nchunks > 1) {
      hipLaunchKernelGGL(gae_carry_kernel<true>, cgrid, dim3(cp.Ew * cp.Rw), 0, stream, a.summary,
                         const_cast<double*>(a.carry), a.chunk_sum, p.Tt, a.N, cp.Ew, cp.Rw,
                         cp.nchunks);
      if ((st = last_launch_status())) return st;
    }
    hipLaunchKernelGGL(gae_carry_kernel<false>, cgrid, dim3(cp.Ew * cp.Rw), 0, stream, a.summary,
                       const_cast<double*>(a.carry), a.chunk_sum, p.Tt, a.N, cp.Ew, cp.Rw,
                       cp.nchunks);
    if ((st = last_launch_status())) return st;
    if (!norm) {
      const PassGeom& gf = p.final_geom(false);
      return launch_tile(tile_kernel<kFinal>(p.vw, gf), gf, a, p.Tt, stream);
    }
    // the final pass writes adv and ret and leaves fp64 (n, sum, sum of
    // squares) of its fp32 advantages per block; then the elementwise
    // normaliser.  (The tile passes used to carry closed-form fp32 sums of
    // each tile's suffix composites into the carry scan, saving the
    // normaliser's re-read; their rounding lost the variance once |mean|
    // exceeded ~100 std.)
    if ((st = launch_tile(tile_kernel<kFinalPartials>(p.vw, p.fin), p.fin, a, p.Tt, stream)))
      return st;
    return launch_normalize(a.partial, p.Tt * p.fin.Tq, a.eps, a.adv, a.adv_n, a.T * a.N, a.hdr,
                            a.stats_out, stream);
  }
  a.carry = nullptr;
  if (!norm) {
    const PassGeom& gf = p.final_geom(false);
    return launch_tile(tile_kernel<kFinal>(p.vw, gf), gf, a, p.Tt, stream);
  }
  // single-tile horizon: partials from the final pass, then the elementwise normaliser
  if ((st = launch_tile(tile_kernel<kFinalPartials>(p.vw, p.fin), p.fin, a, p.Tt, stream)))
    return st;
  return launch_normalize(a.partial, p.Tt * p.fin.Tq, a.eps, a.adv, a.adv_n, a.T * a.N, a.hdr,
                          a.stats_out, stream);
}

// Narrow rollouts without the normaliser (16 <= N < 1024) take the
// one-env-per-thread tiles even when aligned: measured 10-13% faster for
// N = 16-256 (T x N = 2^20 x 16: 107.7 -> 97.4 us), while N = 4 is 40% slower.
bool narrow_scalar(long T, long N, bool norm) { return !norm && N >= 16 && N / 4 < kBlock; }

// Aligned rollouts too narrow for the strip walk take the span passes when
// normalising or narrower than 64 envs (measured on MI355X, us, span vs tile
// passes: N=4 x T=4M 92 vs 250, N=16 x T=1M 87 vs 98; with the normaliser
// 122 vs 411, 118 vs 145, and 117-122 vs 122-125 for N = 64-1024; without it
// N = 64-1024 are within 2%, and below 2^20 elements the tile passes'
// launches are ~1.5 us shorter).
bool span_route(long T, long N, bool norm) {
  return PPO_GAE_SPAN && span_plan(T, N, kSpanMaxBlocks).E > 0 &&
         strip_plan(make_plan(T, N, 4)).E == 0 && (norm || (N < 64 && T * N >= (1L << 20)));
}

int gae_impl(const float* rewards, const float* values, const uint8_t* dones,
             const float* last_value, int64_t T, int64_t N, double gamma, double lam, double eps,
             float* adv_out, float* ret_out, float* adv_norm_out, float* stats_out, bool norm,
             void* workspace, size_t workspace_bytes, void* stream_ptr) {
  if (T < 0 || N < 0) return PPO_ERR_INVALID_ARG;
  if (T == 0 || N == 0) return PPO_OK;
  if (!rewards || !dones || !adv_out) return PPO_ERR_INVALID_ARG;
  if (norm && !adv_norm_out) return PPO_ERR_INVALID_ARG;
  if (N > (1L << 31) || T > (1L << 40) || T * N > (1L << 50)) return PPO_ERR_TOO_LARGE;
  if (!workspace || workspace_bytes < ppo_gae_workspace_bytes(T, N)) return PPO_ERR_WORKSPACE;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);

  const bool vec = (N % 4 == 0) && aligned(rewards, 16) && (!values || aligned(values, 16)) &&
                   aligned(adv_out, 16) && (!ret_out || aligned(ret_out, 16)) &&
                   aligned(dones, 4) && (!last_value || aligned(last_value, 16));
  const GaePlan p = make_plan(T, N, vec && !narrow_scalar(T, N, norm) ? 4 : 1);
  if (p.blocks() > 0x7fffffffL || make_carry_plan(p.Tt, N).nchunks > 65535)
    return PPO_ERR_TOO_LARGE;
  const GaeLayout l = make_layout(p, N);
  char* ws = static_cast<char*>(workspace);

  GaeArgs a = {};
  a.r = rewards;
  a.v = values;
  a.d = dones;
  a.lastv = last_value;
  a.T = T;
  a.N = N;
  a.gamma = gamma;
  a.gl = gamma * lam;
  a.adv = adv_out;
  a.ret = ret_out;
  a.summary = reinterpret_cast<double2*>(ws + l.summary);
  a.carry = reinterpret_cast<double*>(ws + l.carry);
  a.chunk_sum = reinterpret_cast<double2*>(ws + l.chunk_sum);
  a.partial = reinterpret_cast<double*>(ws + l.partial);
  a.hdr = reinterpret_cast<WsHeader*>(ws);
  a.stats_out = stats_out;
  a.eps = eps;
  a.adv_n = adv_norm_out;
  a.slots = reinterpret_cast<uint64_t*>(ws + l.slots);

  // Aligned rollouts whose tiles all fit on the device at once take the
  // resident pass (one read of the rollout, one write of each output).
  if (vec && (!norm || aligned(adv_norm_out, 16))) {
    const int st = launch_resident(T, N, a, norm, stream);
    if (st >= 0) return st;
  }

  if (vec && span_route(T, N, norm)) return launch_span(T, N, a, norm, stream);
  return launch_gae(p, a, norm, stream);
}

}  // namespace
}  // namespace ppo

extern "C" int ppo_gae_route(int64_t T, int64_t N, int normalize, int has_values) {
  using namespace ppo;
  if (T <= 0 || N <= 0) return PPO_GAE_ROUTE_NONE;
  const bool norm = normalize != 0;
  if (N > (1L << 31) || T > (1L << 40) || T * N > (1L << 50)) return PPO_GAE_ROUTE_NONE;
  const bool vec = N % 4 == 0;
  if (vec && resident_ok(T, N, norm, has_values != 0)) return PPO_GAE_ROUTE_RESIDENT;
  if (vec && span_route(T, N, norm)) return PPO_GAE_ROUTE_SPAN;
  const GaePlan p = make_plan(T, N, vec && !narrow_scalar(T, N, norm) ? 4 : 1);
  return strip_plan(p).E > 0 ? PPO_GAE_ROUTE_STRIP : PPO_GAE_ROUTE_TILES;
}

extern "C" size_t ppo_gae_workspace_bytes(int64_t T, int64_t N) {
  using namespace ppo;
  if (T <= 0 || N <= 0) return kHeaderBytes;
  size_t b = make_layout(make_plan(T, N, 1), N).total;
  if (N % 4 == 0) b = std::max(b, make_layout(make_plan(T, N, 4), N).total);
  return b;
}

extern "C" int ppo_gae_f32(const float* rewards, const float* values, const uint8_t* dones,
                           const float* last_value, int64_t T, int64_t N, double gamma,
                           double lam, float* adv_out, float* ret_out, void* workspace,
                           size_t workspace_bytes, void* stream) {
  return ppo::gae_impl(rewards, values, dones, last_value, T, N, gamma, lam, 0.0, adv_out,
                       ret_out, nullptr, nullptr, false, workspace, workspace_bytes, stream);
}

extern "C" int ppo_gae_norm_f32(const float* rewards, const float* values, const uint8_t* dones,
                                const float* last_value, int64_t T, int64_t N, double gamma,
                                double lam, double eps, float* adv_out, float* ret_out,
                                float* adv_norm_out, float* stats_out, void* workspace,
                                size_t workspace_bytes, void* stream) {
  return ppo::gae_impl(rewards, values, dones, last_value, T, N, gamma, lam, eps, adv_out,
                       ret_out, adv_norm_out, stats_out, true, workspace, workspace_bytes,
                       stream);
}

#ifdef PPO_GAE_RES_TRACE
extern "C" __attribute__((visibility("default"))) void* ppo_debug_res_trace(void) {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(ppo::g_res_trace)) != hipSuccess) return nullptr;
  return p;
}
#endif
