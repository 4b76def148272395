// Single-pass linear-recurrence scan with decoupled look-back, for gfx950.
//
// One kernel template serves the scalar scan (philtorch::recur / lti_recur)
// and the 2x2 scan (recur2 / lti_recur2), forward (REV=false) and the fused
// adjoint backward (REV=true).
//
// Work decomposition (per tile of one batch row; tiles never span rows):
//   * a workgroup is W data waves, plus one look-back wave for some
//     algebras; a data wave owns a contiguous segment of 64*K*R steps;
//   * the segment is read in R "rounds" of 64*K contiguous steps, lane l
//     holding steps [l*K, l*K+K) of the round, so every vector load/store of
//     a round is one contiguous 64*K*sizeof(step) byte run (K*sizeof(state)
//     is 16 B or more: one dwordx4 per lane and array);
//   * pass 1: each lane folds its K steps into one affine map; a wave64
//     DPP scan (row_shr 1/2/4/8, row_bcast 15/31, wave_shr 1) turns lane
//     maps into exclusive maps; rounds are chained inside the wave; the W
//     wave aggregates meet in LDS;
//   * look-back (the extra wave, or data wave 0 where the algebra has no
//     look-back wave): it combines the wave aggregates, publishes
//     the tile's aggregate map, then reads the status entries of its 64
//     nearest predecessors, which are contiguous, with coalesced loads (64
//     consecutive words per instruction), stages them in LDS, and lane i
//     takes the entry of tile q-1-i; the nearest predecessor with an
//     inclusive state ends the search and the aggregates in between are
//     reduced in one wave operation;
//   * pass 2: each lane re-runs its K steps from its now-known entry state and
//     writes results with vector stores.
//
// Status words: every 32-bit chunk of a published value is one 64-bit word
// (tag<<32 | chunk) written with an agent-scope atomic store.  A reader
// accepts a value only when every one of its words carries this call's tag,
// so payload and flag can never tear and no fence is needed.
//
// Self-resetting workspace: the workspace starts with kStripes 64-bit claim
// words {epoch (high 32 bits), claim count (low 32 bits)}, one per 128-byte
// line.  Workgroup g claims from stripe g % kStripes with one atomic add,
// which returns its claim index c and the epoch (the grid is padded to whole
// stripes, surplus workgroups exit).  Its tile is g itself (workgroups are
// dispatched in index order), except in the 2x2 time-varying backward, which
// takes c*kStripes + g%kStripes, the order of the claims.  Striping keeps
// same-address atomics from serialising the launch.  The call
// tags its status words with epoch+1.  The last claimer of each stripe
// re-arms it with {epoch+1, 0}: every claim on that stripe has happened by
// then.  Words left by earlier calls carry older tags and are ignored, so the
// workspace is zero-filled only when allocated (and by its owner again every
// 2^31 calls, before the 32-bit tags could repeat); no clearing kernel and no
// end-of-kernel bookkeeping run per call.  Consecutive calls sharing a
// workspace must be stream-ordered.
//
// Forward progress does not depend on the order in which the hardware starts
// workgroups: the look-back polls a bounded number of times, and a tile whose
// predecessors have not all published by then computes its entry state
// itself, folding every earlier step of its row straight from the inputs.
// Tiles are mapped q-major (id = q*B + b), so in practice predecessors start
// first and that path is only taken by the tests that force it.
#pragma once

#include <type_traits>

#include "phs_algebra.hpp"

namespace phs {

constexpr size_t gcd16(size_t n) { return n % 16 == 0 ? 16 : n % 8 == 0 ? 8 : n % 4 == 0 ? 4 : n % 2 == 0 ? 2 : 1; }

// Per-tile status record of the look-back: an inclusive prefix and an
// aggregate map in 64-bit (tag, word) pairs.  Independent of the tile shape.
template <class Alg>
struct StatusShape {
  static constexpr int kIncWords = sizeof(typename Alg::state) / 4;
  static constexpr int kAggWords = sizeof(Map<Alg>) / 4;
  static constexpr int kStride = kIncWords + kAggWords;  // 64-bit words per tile
  // LDS staging of a 64-tile look-back window: one entry per tile, padded to
  // an odd number of words so that lanes reading successive entries spread
  // over the banks
  static constexpr int kLookPitch = kStride | 1;
  static constexpr int kLookWords = 64 * kLookPitch;
};

// Tile shape of one scan mode (TV: per-step coefficients; LTI: one
// coefficient per row).  LTI scans load no coefficients, so their lanes can
// carry more steps in the same registers (Alg::kVecsPerLaneLTI).
template <class Alg, bool TV>
struct Shape : StatusShape<Alg> {
  static constexpr int kWaves = Alg::kWavesPerBlock;  // data waves
  static constexpr bool kLookbackWave = Alg::kLookbackWave;
  static constexpr int kThreads = 64 * (kWaves + (kLookbackWave ? 1 : 0));
  using state = typename Alg::state;
  using s_state = typename Alg::s_state;
  // steps per lane and round: a whole number of 16-byte vectors of stored
  // states, kVecs vectors' worth where a state is under 16 bytes
  static constexpr int kVecs = TV ? Alg::kVecsPerLane : Alg::kVecsPerLaneLTI;
  static constexpr int kMinSteps = 16 / int(gcd16(sizeof(s_state)));  // smallest K with K*size % 16 == 0
  static constexpr int K = sizeof(s_state) >= 16 || kVecs * 16 < int(kMinSteps * sizeof(s_state))
                               ? kMinSteps
                               : kVecs * int(16 / sizeof(s_state)) / kMinSteps * kMinSteps;
  static_assert(K >= 1 && (K * sizeof(s_state)) % 16 == 0, "chunks must be whole 16-byte vectors");
  static constexpr int R = Alg::kRounds;
  static constexpr int kWaveSeg = 64 * K * R;
  static constexpr int kTile = kWaves * kWaveSeg;
  static_assert(kWaves >= 1 && kWaves <= 16, "1..16 waves per workgroup");
};

template <class Alg>
struct ScanArgs {
  using T = typename Alg::elem;
  const T *coef;            // TV: row-major [rows, T, coef]; LTI: [rows, coef]
  int64_t coef_row_stride;  // in coefficients between batch rows (0 = shared)
  const T *zi;              // [B, state]
  const T *x;               // forward: input x;  backward: upstream grad g
  const T *y;               // backward: forward output y
  T *out;                   // forward: y;  backward: grad_x (nullable)
  T *gcoef;                 // backward, TV: per-step coefficient grad (nullable)
  void *partials;           // backward, LTI: per-tile coefficient-grad sums (nullable)
  T *gzi;                   // backward: grad of zi (nullable)
  int64_t B, T_len, tiles_per_row;
  unsigned long long *claims;  // kStripes claim words, 128 bytes apart (workspace offset 0)
  // look-back wave: polls allowed before the tile's own aggregate is known
  // (0: wait for it; the host enables early polling when a row's
  // predecessor tile is claimed a whole resident grid earlier)
  unsigned early_polls;
  unsigned tiles;              // B * tiles_per_row
  unsigned per_stripe;         // claims per stripe (grid = per_stripe * kStripes)
  unsigned spin_limit;         // look-back polls before the self-compute fallback
  unsigned agg_only;           // testing: tiles after a row's first publish no inclusive state
  // tile id -> (scan position, row) without a 64-bit division: for ids
  // below 2^31, id / B == (id * b_magic) >> b_shift (set by the host)
  uint64_t b_magic;
  unsigned b_shift;
  uint64_t *status;          // status words of this call
  int vec_ok;
  // tracing launches only (scan_kernel<..., TRACE = true>): per-tile phase
  // records, kTraceWords 64-bit words per tile id, for ids below trace_tiles
  uint64_t *trace;
  unsigned trace_tiles;
};

// Per-tile phase record of a tracing launch (phs_debug_trace_next_launch):
// s_memrealtime stamps (a constant 100 MHz clock shared by the whole chip)
// at the workgroup's start, after its tile claim, when data wave 0 has
// loaded and folded its segment, when the tile's wave aggregates are in
// (the look-back starts), when its entry state is known, and when data wave
// 0 has issued its last stores; then the look-back's failed polls and the
// tile id.
constexpr int kTraceWords = 8;
enum TraceSlot { kTrStart, kTrClaimed, kTrLoaded, kTrAggregates, kTrEntry, kTrStored, kTrPolls, kTrId };

__device__ __forceinline__ uint64_t trace_clock() { return __builtin_amdgcn_s_memrealtime(); }

constexpr int kStripes = 16;
constexpr int kStripeWords = 16;  // 128 bytes between claim words
constexpr size_t kHeaderBytes = kStripes * kStripeWords * sizeof(unsigned long long);

__device__ __forceinline__ void claim_tile(unsigned long long *claims, unsigned per_stripe, unsigned &id,
                                           unsigned &tag) {
  const unsigned j = blockIdx.x % kStripes;
  unsigned long long *w = claims + j * kStripeWords;
  const unsigned long long v = __hip_atomic_fetch_add(w, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned epoch = unsigned(v >> 32), c = unsigned(v);
  id = c * kStripes + j;
  tag = epoch + 1u;
  if (c == per_stripe - 1u)
    __hip_atomic_store(w, (unsigned long long)(epoch + 1u) << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The call's tag for a workgroup whose tile is its own index (kernels with a
// look-back wave: the data waves load at once, the look-back wave claims
// from the stripe, which counts the workgroup for the re-arming and gives the
// tag).  Called by the whole look-back wave; lane 0 claims.
__device__ __forceinline__ unsigned claim_tag(unsigned long long *claims, unsigned per_stripe, int lane) {
  unsigned cid = 0, ctag = 0;
  if (lane == 0) claim_tile(claims, per_stripe, cid, ctag);
  return __builtin_amdgcn_readfirstlane(ctag);
}

// The same claim split in two for a workgroup whose tile is its own index
// and whose data wave 0 looks back: the atomic is issued before the tile's
// loads and its result is read only at the look-back, so its round trip
// overlaps the loads.  claim_issue: one lane; claim_finish: the whole wave
// (lane 0 holds the claim word), returns the tag and re-arms the stripe if
// this was its last claim.
__device__ __forceinline__ unsigned long long claim_issue(unsigned long long *claims) {
  return __hip_atomic_fetch_add(claims + (blockIdx.x % kStripes) * kStripeWords, 1ull, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned claim_finish(unsigned long long *claims, unsigned per_stripe,
                                                 unsigned long long v, int lane) {
  unsigned tag = 0;
  if (lane == 0) {
    const unsigned epoch = unsigned(v >> 32), c = unsigned(v);
    tag = epoch + 1u;
    if (c == per_stripe - 1u)
      __hip_atomic_store(claims + (blockIdx.x % kStripes) * kStripeWords, (unsigned long long)(epoch + 1u) << 32,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return __builtin_amdgcn_readfirstlane(tag);
}

// (q, b) of tile id = q * B + b with the host's row_split constants.
__device__ __forceinline__ void split_tile(int64_t id, int64_t B, uint64_t magic, unsigned shift, int64_t &q,
                                           int64_t &b) {
  const unsigned uq = unsigned((uint64_t(unsigned(id)) * magic) >> shift);
  q = uq;
  b = int64_t(unsigned(id) - uq * unsigned(B));
}

// ------------------------------------------------------------ status words
template <typename X>
__device__ __forceinline__ void publish(uint64_t *dst, const X &v, unsigned tag) {
  constexpr int n = sizeof(X) / 4;
  union {
    X x;
    uint32_t w[n];
  } u;
  u.x = v;
#pragma unroll
  for (int i = 0; i < n; ++i)
    __hip_atomic_store(dst + i, (uint64_t(tag) << 32) | uint64_t(u.w[i]), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Decodes a value from status words already read; true when every word
// carries `tag`.
template <typename X>
__device__ __forceinline__ bool unpack(const uint64_t *src, X &v, unsigned tag) {
  constexpr int n = sizeof(X) / 4;
  union {
    X x;
    uint32_t w[n];
  } u;
  bool ok = true;
#pragma unroll
  for (int i = 0; i < n; ++i) {
    const uint64_t word = src[i];
    ok = ok & (unsigned(word >> 32) == tag);
    u.w[i] = uint32_t(word);
  }
  v = u.x;
  return ok;
}

// Orders one wave's LDS accesses across its lanes (LDS operations of a wave
// execute in issue order; the fences keep the compiler from moving them).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ------------------------------------------------------------ coalesced stores
// A lane that owns K consecutive steps writes them as NV 16-byte vectors of
// its own, so one store instruction of the wave touches 64 separate
// segments.  Through a lane-blocked LDS buffer of the wave (64 NV vectors)
// the same block leaves as NV instructions of 64 consecutive vectors each
// (1 KB in one piece).  Slot swizzle: block lane L's vector v sits at
// L NV + (v ^ lds_swizzle<NV>(L)), so both the lanes' writes of one vector
// and the reads of 64 consecutive vectors fall in distinct banks within
// each group of 16 lanes.
template <int NV>
__device__ __forceinline__ int lds_swizzle(int L) {
  static_assert(NV >= 1 && NV <= 16 && (NV & (NV - 1)) == 0, "a power of two up to 16");
  constexpr int p = NV >= 16 ? 4 : NV >= 8 ? 3 : NV >= 4 ? 2 : NV >= 2 ? 1 : 0;
  return (L >> (4 - p)) & (NV - 1);
}

// NV vectors a lane, block lane count 64 and a power of two up to 16.
template <typename X, int K>
constexpr bool kLdsBlocked = int(K * sizeof(X)) % 16 == 0 && int(K * sizeof(X) / 16) > 1 &&
                             int(K * sizeof(X) / 16) <= 16 && (int(K * sizeof(X) / 16) & (int(K * sizeof(X) / 16) - 1)) == 0;

// Block lane L's chunk (ascending) into the wave's buffer.
template <typename X, int K>
__device__ __forceinline__ void lds_put_chunk(uint4 *wb, int L, const X (&v)[K]) {
  constexpr int NV = int(K * sizeof(X) / 16);
  union {
    X x[K];
    uint4 u[NV];
  } t;
#pragma unroll
  for (int k = 0; k < K; ++k) t.x[k] = v[k];
  const int sw = lds_swizzle<NV>(L);
#pragma unroll
  for (int i = 0; i < NV; ++i) wb[L * NV + (i ^ sw)] = t.u[i];
}

// The wave's buffer to its block at dst (16-byte aligned, in range): vector
// c of the block is block lane c / NV's vector c % NV.
template <int NV>
__device__ __forceinline__ void lds_flush(uint4 *dst, const uint4 *wb, int lane, bool write) {
  wave_sync();
  if (write) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = j * 64 + lane, L = c / NV, v = c % NV;
      dst[c] = wb[L * NV + (v ^ lds_swizzle<NV>(L))];
    }
  }
  wave_sync();  // later writes to the buffer follow these reads
}

// Wave-level look-back.  `row_status` points at tile 0 of this row's status;
// `virt` is the state entering the row (zi forward, 0 backward); `s_look` is
// LDS for one window.
//
// A window is the n = min(64, base+1) tiles [base+1-n, base]; their entries
// are the words [(base+1-n)*kStride, (base+1)*kStride) of the row, read 64
// consecutive words per instruction from one base address.  (Reading
// entry-per-lane instead costs 64 separate requests per word and competes
// with the co-resident tiles' data loads.)

// Progress of one tile's look-back, kept across polls.
template <class Alg>
struct Lookback {
  Map<Alg> acc;    // fold of the windows already passed
  int64_t base;    // newest tile of the current window
  unsigned polls;  // polls that found some predecessor still unpublished
  int span;        // tiles per window: Alg::kLookFirst first, then 64
};

// The first window reads Alg::kLookFirst entries: a full window is 64
// entries of status words, read again at every poll, and where the nearest
// inclusive predecessor is usually close a narrow first read saves most of it.
template <class Alg>
__device__ __forceinline__ Lookback<Alg> lookback_start(int64_t q) {
  static_assert(Alg::kLookFirst >= 1 && Alg::kLookFirst <= 64, "a window is at most one wave of entries");
  return {map_identity<Alg>(), q - 1, 0u, Alg::kLookFirst};
}

// One poll.  When every tile between the nearest inclusive predecessor and
// this tile has published its aggregate, stores the state entering the tile
// in `out` and returns true (a window of aggregates only is folded into
// lb.acc and the next window read straight away).  Otherwise counts the poll
// and returns false.
template <class Alg>
__device__ bool lookback_poll(const uint64_t *row_status, const typename Alg::state &virt, int lane,
                              unsigned tag, uint64_t *s_look, Lookback<Alg> &lb, typename Alg::state &out) {
  using S = typename Alg::state;
  using M = Map<Alg>;
  using Sh = StatusShape<Alg>;
  constexpr int kS = Sh::kStride, kP = Sh::kLookPitch;
  constexpr int kBatch = kS < 8 ? kS : 8;  // words in flight per lane
  while (true) {
    const int64_t base = lb.base;
    const int n = base + 1 > lb.span ? lb.span : int(base + 1);  // tiles in the window
    const uint64_t *win = row_status + (base + 1 - n) * kS + lane;
    const int64_t p = base - lane;  // lane < n: window entry n-1-lane
    M mv = map_identity<Alg>();
    S sv = Alg::szero();
    // all loads of a batch are issued before any LDS store: atomic loads are
    // ordered against other memory operations, so interleaving them with the
    // stores would serialise one round trip per word
#pragma unroll
    for (int i0 = 0; i0 < kS; i0 += kBatch) {
      uint64_t words[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        words[i] = 0;
        if (i0 + i < kS && (i0 + i) * 64 + lane < n * kS)  // word (i0+i)*64+lane of the window
          words[i] = __hip_atomic_load(win + (i0 + i) * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int j = (i0 + i) * 64 + lane;
        if (i0 + i < kS) s_look[(j / kS) * kP + (j % kS)] = words[i];
      }
    }
    wave_sync();
    // st: 2 inclusive (or the row's virtual entry at p = -1), 1 aggregate
    // only, 0 unpublished, 3 outside the window (identity, never inclusive)
    int st = 3;
    if (lane < n) {
      const uint64_t *e = s_look + (n - 1 - lane) * kP;
      const bool inc_ok = unpack(e, sv, tag);
      const bool agg_ok = unpack(e + Sh::kIncWords, mv, tag);
      st = inc_ok ? 2 : (agg_ok ? 1 : 0);
      if (!agg_ok) mv = map_identity<Alg>();
    } else if (p == -1) {
      st = 2;
      sv = virt;
    }
    wave_sync();
    const uint64_t incm = __ballot(st == 2);
    const int k = incm ? __builtin_ctzll(incm) : 64;
    const uint64_t low = (k >= 64) ? ~0ull : ((1ull << k) - 1ull);
    if (__ballot(st == 0) & low) {
      ++lb.polls;
      return false;
    }
    // lanes [0, k) hold aggregates of tiles base-lane (newest at lane 0);
    // fold them oldest-first into lane 0 (lanes outside the window carry the
    // identity).
    M m = (lane < k) ? mv : map_identity<Alg>();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      M o = shfl_from(m, lane + d);
      if (lane + d < 64) m = compose<Alg>(o, m);
    }
    const M F = read_lane(m, 0);
    if (k < 64) {
      const S yk = read_lane(sv, k);
      out = apply<Alg>(compose<Alg>(F, lb.acc), yk);
      return true;
    }
    lb.acc = compose<Alg>(F, lb.acc);
    lb.base = base - n;
    lb.span = 64;
  }
}

// Blocking look-back: polls until the entry state is known (true), or
// returns false once lb.polls reaches spin_limit.
template <class Alg>
__device__ bool lookback(const uint64_t *row_status, const typename Alg::state &virt, int lane, unsigned tag,
                         unsigned spin_limit, uint64_t *s_look, Lookback<Alg> &lb, typename Alg::state &out) {
  while (!lookback_poll<Alg>(row_status, virt, lane, tag, s_look, lb, out)) {
    if (lb.polls >= spin_limit) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

// ------------------------------------------------------------ chunk I/O
// The bounds-checked tail assigns in branches: `c ? row[t] : fill` with both
// operands lvalues is an lvalue, compiled as a select between a global and a
// private address, and every thread of the kernel then keeps a copy of
// `fill` in scratch memory.  kFull: the caller knows the chunk is in range
// and 16-byte aligned, so only the vector path is compiled (no branch
// between the forms; see the kernel's full-tile path).
template <typename X, int K, bool kFull = false>
__device__ __forceinline__ void load_chunk(const X *row, int64_t t0, int64_t T, bool vec, X (&out)[K],
                                           const X fill) {
  if (kFull || (vec && t0 + K <= T)) {
    constexpr int nv = int(K * sizeof(X) / 16);
    static_assert(K * sizeof(X) % 16 == 0, "chunk must be 16-byte granular");
    union {
      X x[K];
      uint4 v[nv];
    } u;
    const uint4 *p = reinterpret_cast<const uint4 *>(row + t0);
#pragma unroll
    for (int i = 0; i < nv; ++i) u.v[i] = p[i];
#pragma unroll
    for (int k = 0; k < K; ++k) out[k] = u.x[k];
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      if (t0 + k < T)
        out[k] = row[t0 + k];
      else
        out[k] = fill;
    }
  }
}

template <typename X, int K, bool kFull = false>
__device__ __forceinline__ void store_chunk(X *row, int64_t t0, int64_t T, bool vec, const X (&v)[K]) {
  if (kFull || (vec && t0 + K <= T)) {
    constexpr int nv = int(K * sizeof(X) / 16);
    union {
      X x[K];
      uint4 v[nv];
    } u;
#pragma unroll
    for (int k = 0; k < K; ++k) u.x[k] = v[k];
    uint4 *p = reinterpret_cast<uint4 *>(row + t0);
#pragma unroll
    for (int i = 0; i < nv; ++i) p[i] = u.v[i];
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (t0 + k < T) row[t0 + k] = v[k];
  }
}

// A lane's K steps folded into one map: in storage precision (the error of
// a handful of steps is a few ulps), then widened for every later level.
// Forward step t is (A[t], x[t]); backward it is (A[t]^H, A[t]^H g[t]) and the
// lane walks its chunk downwards.
template <class Alg, bool TV, bool REV, int K>
__device__ __forceinline__ Map<Alg> lane_map(const typename Alg::s_coef (&Ac)[TV ? K : 1],
                                             const typename Alg::s_state (&Xc)[K],
                                             const typename Alg::s_coef &a_row) {
  using SC = typename Alg::s_coef;
  using SS = typename Alg::s_state;
  const SS zero_ss = Alg::s_szero();
  SMap<Alg> f;
#pragma unroll
  for (int kk = 0; kk < K; ++kk) {
    const int k = REV ? K - 1 - kk : kk;
    const SC raw = TV ? Ac[TV ? k : 0] : a_row;
    const SC c = REV ? Alg::s_adjoint(raw) : raw;
    const SS e = REV ? Alg::s_affine(c, Xc[k], zero_ss) : Xc[k];
    if (kk == 0) {
      f.A = c;
      f.x = e;
    } else {
      f.A = Alg::s_cmul(c, f.A);
      f.x = Alg::s_affine(c, f.x, e);
    }
  }
  Map<Alg> m;
  m.A = Alg::load_c(f.A);
  m.x = Alg::load_s(f.x);
  return m;
}

// ------------------------------------------------------------ look-back fallback
// State entering tile (scan position qs) of a row, folded straight from the
// inputs: every step of the row that precedes the tile in scan order, 64*K
// steps per wave iteration.  Taken only when predecessors did not publish
// within the poll budget; kept out of line so that this cold loop does not
// shape the register allocation and schedule of the hot path.
template <class Alg, bool TV, bool REV>
__device__ __noinline__ typename Alg::state row_prefix_fallback(const typename Alg::s_state *xrow,
                                                               const typename Alg::s_coef *crow, int64_t T,
                                                               bool vec, int64_t span, int64_t row_end,
                                                               int lane, typename Alg::state virt) {
  using SC = typename Alg::s_coef;
  using SS = typename Alg::s_state;
  using M = Map<Alg>;
  constexpr int K = Shape<Alg, TV>::K;
  auto op = [](const M &p, const M &q) { return compose<Alg>(p, q); };
  const SC zero_sc = Alg::s_czero();
  const SS zero_ss = Alg::s_szero();
  const SC a_row_s = TV ? zero_sc : crow[0];
  M acc = map_identity<Alg>();
  for (int64_t off = 0; off < span; off += 64 * K) {
    const int64_t c0 = REV ? row_end - off - int64_t(lane + 1) * K : off + int64_t(lane) * K;
    SS xs[K];
    SC cs[TV ? K : 1];
    load_chunk<SS, K>(xrow, c0, T, vec, xs, zero_ss);
    if constexpr (TV) load_chunk<SC, K>(crow, c0, T, vec, cs, zero_sc);
    M m = lane_map<Alg, TV, REV, K>(cs, xs, a_row_s);
    m = wave_scan_incl(m, lane, op);
    acc = compose<Alg>(acc, read_lane(m, 63));
  }
  return apply<Alg>(acc, virt);
}

// The running kernel's argument block where it lies in the kernarg segment
// (a kernel whose one parameter is an Args).  Out-of-line cold paths take it
// by this pointer: a by-value copy of a large argument struct is spilled to
// scratch by every wave on entry, on the hot path.
template <class Args>
__device__ __forceinline__ const Args *kernel_args() {
  return (const Args *)__builtin_amdgcn_kernarg_segment_ptr();
}

// ------------------------------------------------------------ tile look-back
// The tile's aggregate: the wave aggregates of s_wagg folded in wave order.
template <class Alg, int kWaves>
__device__ __forceinline__ Map<Alg> tile_aggregate(const Map<Alg> *s_wagg) {
  Map<Alg> t = s_wagg[0];
#pragma unroll
  for (int j = 1; j < kWaves; ++j) t = compose<Alg>(t, s_wagg[j]);
  return t;
}

// State entering tile qs of row b (scan order), found by one wave after the
// tile's aggregate `tagg` is known: publish it, look back over the
// predecessors (or fold the row prefix from the inputs once the poll budget
// is spent), publish the inclusive state.  `known`: the state is already in
// `yin` (the row's first tile, or an early look-back that resolved).  `virt`:
// the state entering the row (zi forward, zero backward).
template <class Alg, bool TV, bool REV>
__device__ __forceinline__ typename Alg::state tile_entry(const ScanArgs<Alg> &a, int64_t qs, int64_t b,
                                                          unsigned tag, int lane, const Map<Alg> &tagg, bool known,
                                                          typename Alg::state yin, Lookback<Alg> &lb,
                                                          uint64_t *s_look, const typename Alg::state &virt) {
  using SC = typename Alg::s_coef;
  using SS = typename Alg::s_state;
  using Sh = Shape<Alg, TV>;
  uint64_t *row_status = a.status + b * a.tiles_per_row * Sh::kStride;
  if (!known) {
    if (!lookback<Alg>(row_status, virt, lane, tag, a.spin_limit, s_look, lb, yin))
      yin = row_prefix_fallback<Alg, TV, REV>(reinterpret_cast<const SS *>(a.x) + b * a.T_len,
                                              reinterpret_cast<const SC *>(a.coef) + b * a.coef_row_stride,
                                              a.T_len, a.vec_ok != 0, qs * Sh::kTile, a.tiles_per_row * Sh::kTile,
                                              lane, virt);
  }
  if (qs + 1 < a.tiles_per_row && lane == 0 && !(a.agg_only && qs > 0))
    publish(row_status + qs * Sh::kStride, apply<Alg>(tagg, yin), tag);
  return yin;
}

// ------------------------------------------------------------ the kernel
// TV  : the coefficient varies along time (LPV); otherwise one per row (LTI).
// REV : backward adjoint scan, nu[t] = A[t]^H (g[t] + nu[t+1]), run from the
//       end of the row towards its start; lambda[t] = g[t] + nu[t+1] is
//       grad_x, lambda[t] conj(y[t-1])^T the coefficient grad, nu[0] grad_zi.
//
// Scan order is always ascending in (wave, round, lane); REV mirrors the
// placement of waves, rounds and lanes in memory instead, so one DPP scan
// serves both directions.  Inside a lane's K steps REV walks downwards.
//
// Every output is written after the tile's entry state is known, so a tile
// reads all of its inputs before it writes anything.  Writing the outputs a
// lane's entry state cannot reach early (from the in-wave prefix, before the
// look-back resolves) was measured slower on every real scalar config: the
// early writes mix into the co-resident tiles' reads (C1 backward 14.8 ->
// 16.6 us, C5 fp64 step 1.80 -> 1.85 ms, same-box A/B).
//
// Full tiles (in range and 16-byte aligned) of real scalar scans and of
// every backward run a copy of the data path with
// only vector loads and stores, so the compiler's memory-counter waits see
// one straight-line sequence of loads and each round's fold waits for its
// own vectors only; with the bounds-checked form in the same code it waited
// for every load of the tile before the first fold.
//
// Where the algebra asks for it (Alg::kLookbackWave), the look-back runs in
// a wave of its own that holds no tile data.  Run by data wave 0 instead, its
// staging words and folded maps are live on top of that wave's loaded chunk
// and scan maps; split into roles, the kernel needs the larger of the two
// register sets, not their sum.  That pays where the data path is
// register-heavy (2x2 and complex scans); for real scalar scans a ninth wave
// per tile costs more than it saves.  Either way the waves meet at the same
// barriers: wave aggregates ready, entry state ready (and, backward for LTI,
// the gradient reduction).
//
// TRACE: the instantiation a tracing launch runs; it also writes each
// tile's phase record (kTraceWords words at trace + id * kTraceWords).
template <class Alg, bool TV, bool REV, bool TRACE = false>
__global__ __launch_bounds__((Shape<Alg, TV>::kThreads), Alg::kMinWavesPerEU) void scan_kernel(ScanArgs<Alg> a) {
  using S = typename Alg::state;     // compute type
  using SC = typename Alg::s_coef;   // storage types
  using SS = typename Alg::s_state;
  using M = Map<Alg>;
  using AC = typename Alg::acc_coef;
  using Sh = Shape<Alg, TV>;
  constexpr int K = Sh::K, R = Sh::R, kWaves = Sh::kWaves;

  __shared__ M s_wagg[kWaves];
  __shared__ S s_in;
  __shared__ unsigned s_id, s_tag;
  __shared__ AC s_acc[kWaves];
  __shared__ uint64_t s_look[Sh::kLookWords];
  __shared__ unsigned s_ready;  // data waves whose aggregate is in s_wagg
  // Outputs of whole rounds leave through LDS (lds_flush) where a lane's
  // chunk is more than one 16-byte vector: states (forward y, backward
  // grad_x) and per-step coefficient gradients, one buffer per wave
  constexpr bool kSLds = kLdsBlocked<SS, K>;
  constexpr bool kCLds = TV && REV && kLdsBlocked<SC, K>;
  constexpr int kNVs = kSLds ? int(K * sizeof(SS) / 16) : 1;
  constexpr int kNVc = kCLds ? int(K * sizeof(SC) / 16) : 1;
  constexpr int kNVb = kNVs > kNVc ? kNVs : kNVc;
  __shared__ uint4 s_out[(kSLds || kCLds) ? kWaves * 64 * kNVb : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  // wave index as a scalar: the role branches below are scalar branches, so a
  // wave only ever executes the barriers of its own role
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  [[maybe_unused]] uint64_t tr_start = 0;
  if constexpr (TRACE) tr_start = trace_clock();
  // Tile ids.  The tile is the workgroup's own index: workgroups are
  // dispatched in index order, so a tile's row predecessors start first, as
  // claimed tiles do, and the data waves issue their loads at once instead of
  // after a claim's round trip.  The workgroup still claims from its stripe,
  // which counts it for the stripe's re-arming and gives it the call's tag:
  // the look-back wave claims, or, without one, data wave 0 issues the claim
  // before its loads and reads the result at the look-back.  Measured: C4 op
  // level (2x2 LTI) 8.8 -> 9.6 GSamples/s, C2 +1 %, C3's forward 258 -> 240
  // us; C3's backward (2x2 with a look-back wave, time-varying) ran 452 ->
  // 471 us and keeps the claimed order.
  constexpr bool kStaticIds = !(Sh::kLookbackWave && TV && REV);
  constexpr bool kOwnClaim = kStaticIds && !Sh::kLookbackWave;  // data wave 0 claims
  int64_t id = 0;
  unsigned tag = 0;
  [[maybe_unused]] unsigned long long claim_v = 0;
  if constexpr (kStaticIds) {
    if constexpr (Sh::kLookbackWave) {
      if (tid == 0) s_ready = 0;
      __syncthreads();
    }
    id = blockIdx.x;
    if (id >= a.tiles) {  // padding of the last stripe round: counted, then gone
      if (tid == 0) claim_tile(a.claims, a.per_stripe, s_id, s_tag);
      return;
    }
    if constexpr (kOwnClaim) {
      if (tid == 0) claim_v = claim_issue(a.claims);
    }
  } else {
    if (tid == 0) {
      claim_tile(a.claims, a.per_stripe, s_id, s_tag);
      s_ready = 0;
    }
    __syncthreads();
    if (s_id >= a.tiles) return;  // padding of the last stripe round
    id = s_id;
    tag = s_tag;
  }
  uint64_t *tr = nullptr;  // this tile's phase record (tracing launches)
  if constexpr (TRACE) {
    if (id < a.trace_tiles) tr = a.trace + id * kTraceWords;
    if (tr && tid == 0) {
      tr[kTrStart] = tr_start;
      tr[kTrClaimed] = trace_clock();
      tr[kTrId] = uint64_t(id);
    }
  }
  int64_t qs, b;  // position in scan order, row: id = qs * B + b
  split_tile(id, a.B, a.b_magic, a.b_shift, qs, b);
  const int64_t qf = REV ? a.tiles_per_row - 1 - qs : qs;  // position along time
  const int64_t T = a.T_len;
  const bool vec = a.vec_ok != 0;

  const SS *xrow = reinterpret_cast<const SS *>(a.x) + b * T;
  const SC *crow = reinterpret_cast<const SC *>(a.coef) + b * a.coef_row_stride;
  // Steps past the end of the row load a zero coefficient and a zero input.
  // Forward they follow every valid step, so they only touch the aggregate of
  // the row's last tile, which nobody reads.  Backward they come first, where
  // the carry is zero anyway, and keep it zero.
  const SC zero_sc = Alg::s_czero();
  const SS zero_ss = Alg::s_szero();
  const SC a_row_s = TV ? zero_sc : crow[0];
  auto op = [](const M &p, const M &q) { return compose<Alg>(p, q); };
  // only LTI coefficients reduce their gradient inside the kernel (backward)
  constexpr bool kAcc = REV && !TV;
  const bool want_acc = kAcc && a.partials != nullptr;
  uint64_t *row_status = a.status + b * a.tiles_per_row * Sh::kStride;

  if (Sh::kLookbackWave && w == kWaves) {
    // ================= look-back wave
    if constexpr (kStaticIds) tag = claim_tag(a.claims, a.per_stripe, lane);
    const S virt = REV ? Alg::szero() : Alg::load_s(reinterpret_cast<const SS *>(a.zi)[b]);
    Lookback<Alg> lb = lookback_start<Alg>(qs);
    S yin = virt;
    bool known = qs == 0;
    // The entry state does not depend on this tile: where the predecessor is
    // expected to have finished (a.early_polls > 0), poll while the data
    // waves load and scan, until it is known or their aggregates are all in.
    while (!known && lb.polls < a.early_polls) {
      known = lookback_poll<Alg>(row_status, virt, lane, tag, s_look, lb, yin);
      if (known || __hip_atomic_load(&s_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == unsigned(kWaves))
        break;
      __builtin_amdgcn_s_sleep(1);
    }
    __syncthreads();  // wave aggregates are in s_wagg
    if constexpr (TRACE) {
      if (tr && lane == 0) tr[kTrAggregates] = trace_clock();
    }
    const M tagg = tile_aggregate<Alg, kWaves>(s_wagg);
    if (!known && lane == 0) publish(row_status + qs * Sh::kStride + Sh::kIncWords, tagg, tag);
    yin = tile_entry<Alg, TV, REV>(a, qs, b, tag, lane, tagg, known, yin, lb, s_look, virt);
    if constexpr (TRACE) {
      if (tr && lane == 0) {
        tr[kTrEntry] = trace_clock();
        tr[kTrPolls] = lb.polls;
      }
    }
    if (lane == 0) s_in = yin;
    __syncthreads();  // entry state published to the data waves
    if (want_acc) __syncthreads();  // the data waves' gradient reduction
    return;
  }

  // ================= data waves
  // forward without a look-back wave: the state entering the row, read with
  // the tile's data (data wave 0's look-back needs it; one line per wave,
  // converted only where it is used)
  [[maybe_unused]] SS virt_raw = zero_ss;
  if constexpr (!REV && !Sh::kLookbackWave) virt_raw = reinterpret_cast<const SS *>(a.zi)[b];
  // memory placement of this wave's segment and of this lane's chunk
  const int pw = REV ? kWaves - 1 - w : w;
  const int pl = REV ? 63 - lane : lane;
  const int64_t seg0 = qf * Sh::kTile + int64_t(pw) * Sh::kWaveSeg;
  auto chunk0 = [&](int r) -> int64_t {
    const int pr = REV ? R - 1 - r : r;
    return seg0 + int64_t(pr) * 64 * K + int64_t(pl) * K;
  };
  const SS *yrow_in = reinterpret_cast<const SS *>(a.y) + b * T;
  SS *yrow = REV ? nullptr : reinterpret_cast<SS *>(a.out) + b * T;
  SS *gxrow = (REV && a.out) ? reinterpret_cast<SS *>(a.out) + b * T : nullptr;
  SC *gcrow = (REV && a.gcoef) ? reinterpret_cast<SC *>(a.gcoef) + b * T : nullptr;

  // The data path, compiled twice: kFull for tiles wholly inside the row
  // with aligned rows (vector loads and stores only), and the bounds-checked
  // form for the rest.
  auto data_path = [&](auto full_c) {
    constexpr bool kFull = decltype(full_c)::value;
    // ---- loads (all rounds issued up front)
    SS X[R][K];
    SC A[TV ? R : 1][TV ? K : 1];
    SS Y[REV ? R : 1][REV ? K : 1];
    SS Ylow[REV ? R : 1];  // backward: y[t0-1] below the chunk of lane 63
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t t0 = chunk0(r);
      load_chunk<SS, K, kFull>(xrow, t0, T, vec, X[r], zero_ss);
      if constexpr (TV) load_chunk<SC, K, kFull>(crow, t0, T, vec, A[r], zero_sc);
      if constexpr (REV) {
        load_chunk<SS, K, kFull>(yrow_in, t0, T, vec, Y[r], zero_ss);
        Ylow[r] = zero_ss;
        if (lane == 63) {
          if (t0 == 0)
            Ylow[r] = reinterpret_cast<const SS *>(a.zi)[b];
          else if (kFull || t0 - 1 < T)
            Ylow[r] = yrow_in[t0 - 1];
        }
      }
    }

    // ---- pass 2 of round r from the start state h, writing its outputs
    // backward: y[t0-1] of each round sits in the last step of the next
    // lane's chunk (lanes are mirrored), or below the round for lane 63 (set,
    // by a shuffle, outside the per-lane branches of pass 2)
    SS Ybelow[REV ? R : 1];
    auto pass2 = [&](int r, SS h) -> AC {
      AC acc = Alg::acc_zero();
      const int64_t t0 = chunk0(r);
      // the round's block (lowest time first) and whether it is whole and aligned
      const int64_t blk0 = t0 - int64_t(pl) * K;
      const bool blk_full = kFull || (vec && blk0 + 64 * K <= T);
      uint4 *wb = s_out + w * 64 * kNVb;
      if constexpr (!REV) {
        SS O[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
          h = Alg::s_affine(TV ? A[r][TV ? k : 0] : a_row_s, h, X[r][k]);
          O[k] = h;
        }
        if (kSLds && blk_full) {
          if constexpr (kSLds) {
            lds_put_chunk<SS, K>(wb, pl, O);
            lds_flush<kNVs>(reinterpret_cast<uint4 *>(yrow + blk0), wb, lane, true);
          }
        } else {
          store_chunk<SS, K, kFull>(yrow, t0, T, vec, O);
        }
      } else {
        SS nu = h;
        SS GX[K];
        SC GC[K];
#pragma unroll
        for (int kk = 0; kk < K; ++kk) {
          const int k = K - 1 - kk;
          const SC c = Alg::s_adjoint(TV ? A[r][TV ? k : 0] : a_row_s);
          const SS lam = Alg::s_add(X[r][k], nu);
          GX[k] = lam;
          const SC g = Alg::s_outer(lam, k == 0 ? Ybelow[r] : Y[r][k > 0 ? k - 1 : 0]);
          GC[k] = g;
          if constexpr (kAcc) {
            if (want_acc && (kFull || t0 + k < T)) acc = Alg::acc_add(acc, Alg::load_c(g));
          }
          nu = Alg::s_affine(c, lam, zero_ss);
          if (t0 + k == 0 && a.gzi) reinterpret_cast<SS *>(a.gzi)[b] = nu;
        }
        if (kSLds && blk_full) {
          if constexpr (kSLds) {
            lds_put_chunk<SS, K>(wb, pl, GX);
            lds_flush<kNVs>(reinterpret_cast<uint4 *>(gxrow + blk0), wb, lane, gxrow != nullptr);
          }
        } else if (gxrow) {
          store_chunk<SS, K, kFull>(gxrow, t0, T, vec, GX);
        }
        if constexpr (TV) {
          if (kCLds && blk_full) {
            if constexpr (kCLds) {
              lds_put_chunk<SC, K>(wb, pl, GC);
              lds_flush<kNVc>(reinterpret_cast<uint4 *>(gcrow + blk0), wb, lane, gcrow != nullptr);
            }
          } else if (gcrow) {
            store_chunk<SC, K, kFull>(gcrow, t0, T, vec, GC);
          }
        }
      }
      return acc;
    };

    // ---- pass 1: lane maps, wave scans (each round as soon as its vectors
    // are in), round chaining
    M E[R];  // map from the wave's start to this lane's chunk of round r
    M carry = map_identity<Alg>();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      M m = lane_map<Alg, TV, REV, K>(A[TV ? r : 0], X[r], a_row_s);
      m = wave_scan_incl(m, lane, op);
      const M ex = wave_shift_up(m, lane, map_identity<Alg>());
      const M tot = read_lane(m, 63);
      E[r] = compose<Alg>(carry, ex);
      carry = compose<Alg>(carry, tot);
      if constexpr (REV) {
        Ybelow[r] = shfl_from(Y[r][K - 1], lane + 1);
        if (lane == 63) Ybelow[r] = Ylow[r];
      }
    }
    if constexpr (TRACE) {
      if (tr && tid == 0) tr[kTrLoaded] = trace_clock();
    }
    if (lane == 0) {
      s_wagg[w] = carry;
      if (Sh::kLookbackWave) __hip_atomic_fetch_add(&s_ready, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __syncthreads();  // wave aggregates are in s_wagg
    if (!Sh::kLookbackWave && w == 0) {
      // look-back by data wave 0: publish the tile's aggregate, find its entry
      if constexpr (kOwnClaim) tag = claim_finish(a.claims, a.per_stripe, claim_v, lane);
      if constexpr (TRACE) {
        if (tr && lane == 0) tr[kTrAggregates] = trace_clock();
      }
      const M tagg = tile_aggregate<Alg, kWaves>(s_wagg);
      if (qs > 0 && lane == 0) publish(row_status + qs * Sh::kStride + Sh::kIncWords, tagg, tag);
      Lookback<Alg> lb = lookback_start<Alg>(qs);
      const S virt = REV ? Alg::szero() : Alg::load_s(virt_raw);
      const S yin = tile_entry<Alg, TV, REV>(a, qs, b, tag, lane, tagg, qs == 0, virt, lb, s_look, virt);
      if constexpr (TRACE) {
        if (tr && lane == 0) {
          tr[kTrEntry] = trace_clock();
          tr[kTrPolls] = lb.polls;
        }
      }
      if (lane == 0) s_in = yin;
    }
    // the wave's exclusive prefix in the tile, folded by every wave itself
    M wpre = map_identity<Alg>();
    for (int j = 0; j < w; ++j) wpre = compose<Alg>(wpre, s_wagg[j]);
    __syncthreads();  // entry state is in s_in

    // ---- pass 2 from the entry state
    const S hin = apply<Alg>(wpre, s_in);  // state entering this wave's segment
    AC acc = Alg::acc_zero();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const AC v = pass2(r, Alg::store_s(apply<Alg>(E[r], hin)));
      if constexpr (kAcc) acc = Alg::acc_sum(acc, v);
    }
    if constexpr (TRACE) {
      if (tr && tid == 0) tr[kTrStored] = trace_clock();
    }
    if (want_acc) {
      // deterministic block reduction of the per-tile coefficient gradient
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) acc = Alg::acc_sum(acc, shfl_from(acc, lane ^ d));
      if (lane == 0) s_acc[w] = acc;
      __syncthreads();
      if (tid == 0) {
        AC sum = s_acc[0];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) sum = Alg::acc_sum(sum, s_acc[i]);
        reinterpret_cast<AC *>(a.partials)[b * a.tiles_per_row + qf] = sum;
      }
    }
  };
  // The forwards of algebras with a look-back wave (complex, 2x2, order M)
  // keep the single bounds-checked form: with the vector-only copy beside it
  // they measured slower (C2 forward 0.852 -> 0.861 ms, same-box A/B).
  constexpr bool kSplit = !Sh::kLookbackWave || REV;
  if (kSplit && vec && (qf + 1) * Sh::kTile <= T)
    data_path(std::true_type{});
  else
    data_path(std::false_type{});
}

// ------------------------------------------------------------ helpers
constexpr int kReduceThreads = 256;

// out[i] = sum_{j < count} partials[i*count + j], fixed order, one block per i.
template <class Alg>
__global__ __launch_bounds__(kReduceThreads) void reduce_rows_kernel(const void *partials, int64_t count,
                                                                typename Alg::elem *out) {
  using AC = typename Alg::acc_coef;
  __shared__ AC s[kReduceThreads];
  const AC *p = reinterpret_cast<const AC *>(partials) + blockIdx.x * count;
  AC acc = Alg::acc_zero();
  for (int64_t j = threadIdx.x; j < count; j += kReduceThreads) acc = Alg::acc_sum(acc, p[j]);
  s[threadIdx.x] = acc;
  __syncthreads();
  for (int h = kReduceThreads / 2; h > 0; h >>= 1) {
    if (threadIdx.x < h) s[threadIdx.x] = Alg::acc_sum(s[threadIdx.x], s[threadIdx.x + h]);
    __syncthreads();
  }
  if (threadIdx.x == 0)
    reinterpret_cast<typename Alg::s_coef *>(out)[blockIdx.x] = Alg::store_c(s[0]);
}

// out[t] = sum_b per_step[b, t]  (LPV coefficient shared across the batch).
template <class Alg>
__global__ __launch_bounds__(kReduceThreads) void reduce_batch_kernel(const typename Alg::elem *per_step,
                                                                 int64_t B, int64_t T,
                                                                 typename Alg::elem *out) {
  using SC = typename Alg::s_coef;
  const SC *p = reinterpret_cast<const SC *>(per_step);
  for (int64_t t = blockIdx.x * int64_t(kReduceThreads) + threadIdx.x; t < T;
       t += int64_t(gridDim.x) * kReduceThreads) {
    typename Alg::acc_coef acc = Alg::acc_zero();
    for (int64_t b = 0; b < B; ++b) acc = Alg::acc_add(acc, Alg::load_c(p[b * T + t]));
    reinterpret_cast<SC *>(out)[t] = Alg::store_c(acc);
  }
}

}  // namespace phs
