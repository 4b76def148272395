// Single-pass linear-recurrence scan with decoupled look-back, for gfx950.
//
// One kernel template serves the scalar scan (philtorch::recur / lti_recur)
// and the 2x2 scan (recur2 / lti_recur2), forward (REV=false) and the fused
// adjoint backward (REV=true).
//
// Work decomposition (per tile of one batch row; tiles never span rows):
//   * 256 threads = 4 waves; a wave owns a contiguous segment of 64*K*R steps;
//   * the segment is read in R "rounds" of 64*K contiguous steps, lane l
//     holding steps [l*K, l*K+K) of the round, so every vector load/store of
//     a round is one contiguous 64*K*sizeof(step) byte run (K*sizeof(state)
//     is 16 B or more: one dwordx4 per lane and array);
//   * pass 1: each lane folds its K steps into one affine map; a wave64
//     Hillis-Steele scan (ds_bpermute) turns lane maps into exclusive maps;
//     rounds are chained inside the wave; the 4 wave aggregates meet in LDS;
//   * look-back (wave 0): the tile publishes its aggregate map, then lane i
//     polls the status words of predecessor tile q-1-i; the nearest
//     predecessor with an inclusive state ends the search and the aggregates
//     in between are reduced in one wave operation;
//   * pass 2: each lane re-runs its K steps from its now-known entry state and
//     writes results with vector stores.
//
// Status words: every 32-bit chunk of a published value is one 64-bit word
// (tag<<32 | chunk) written with an agent-scope atomic store.  A reader
// accepts a value only when every one of its words carries this call's tag,
// so payload and flag can never tear and no fence is needed.
//
// Self-resetting workspace: the workspace starts with a header
// {tile counter, finished-block counter, epoch}.  A call tags its words with
// epoch+1; the last workgroup to finish (it sees the finished counter reach
// gridDim-1 after every wave of every block has drained its memory traffic)
// zeroes both counters and stores the new epoch.  Words left by earlier calls
// carry older tags and are ignored, so the workspace needs zero-filling only
// once, when it is allocated, and no clearing kernel runs per call.  When the
// 32-bit tag space wraps, that last workgroup also zeroes the whole status
// area.  Consecutive calls sharing a workspace must be stream-ordered.
//
// Tiles are claimed through an atomic counter in launch order, mapped
// q-major (id = q*B + b): a tile's predecessor always holds a smaller id, so
// it has been claimed by a running or finished workgroup and every wait ends.
#pragma once

#include "phs_algebra.hpp"

namespace phs {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

template <class Alg>
struct Shape {
  using state = typename Alg::state;
  using s_state = typename Alg::s_state;
  // steps per lane and round: one 16-byte vector of stored states (or more)
  static constexpr int K = sizeof(s_state) >= 16 ? 1 : int(16 / sizeof(s_state));
  static constexpr int R = Alg::kRounds;
  static constexpr int kWaveSeg = 64 * K * R;
  static constexpr int kTile = kWaves * kWaveSeg;
  static constexpr int kIncWords = sizeof(state) / 4;
  static constexpr int kAggWords = sizeof(Map<Alg>) / 4;
  static constexpr int kStride = kIncWords + kAggWords;  // 64-bit words per tile
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
  unsigned *header;          // [0] tile counter, [1] finished blocks, [2] epoch
  uint64_t *status;          // status words of this call
  int64_t status_capacity;   // 64-bit words available from `status` on
  int vec_ok;
};

enum : int { kHdrCounter = 0, kHdrDone = 1, kHdrEpoch = 2 };

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

template <typename X>
__device__ __forceinline__ bool try_read(uint64_t *src, X &v, unsigned tag) {
  constexpr int n = sizeof(X) / 4;
  union {
    X x;
    uint32_t w[n];
  } u;
  bool ok = true;
#pragma unroll
  for (int i = 0; i < n; ++i) {
    uint64_t word = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ok = ok & (unsigned(word >> 32) == tag);
    u.w[i] = uint32_t(word);
  }
  v = u.x;
  return ok;
}

// Wave-level look-back.  `row_status` points at tile 0 of this row's status;
// `q` is this tile's position in scan order; `virt` is the state entering
// the row (zi forward, 0 backward).  Returns the state entering tile q.
template <class Alg>
__device__ typename Alg::state lookback(uint64_t *row_status, int64_t q,
                                        const typename Alg::state &virt, int lane, unsigned tag) {
  using S = typename Alg::state;
  using M = Map<Alg>;
  using Sh = Shape<Alg>;
  M acc = map_identity<Alg>();
  int64_t base = q - 1;
  while (true) {
    const int64_t p = base - lane;
    M mv = map_identity<Alg>();
    S sv = Alg::szero();
    int k;
    while (true) {
      int st;
      if (p < 0) {
        st = 2;
        sv = (p == -1) ? virt : Alg::szero();
      } else {
        uint64_t *s = row_status + p * Sh::kStride;
        if (try_read(s, sv, tag))
          st = 2;
        else if (try_read(s + Sh::kIncWords, mv, tag))
          st = 1;
        else
          st = 0;
      }
      const uint64_t incm = __ballot(st == 2);
      k = incm ? __builtin_ctzll(incm) : 64;
      const uint64_t low = (k >= 64) ? ~0ull : ((1ull << k) - 1ull);
      const uint64_t waiting = __ballot(st == 0) & low;
      if (waiting == 0) break;
      __builtin_amdgcn_s_sleep(1);
    }
    // lanes [0, k) hold aggregates of tiles q-1-lane (newest at lane 0);
    // fold them oldest-first into lane 0.
    M m = (lane < k) ? mv : map_identity<Alg>();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      M o = shfl_from(m, lane + d);
      if (lane + d < 64) m = compose<Alg>(o, m);
    }
    const M F = read_lane(m, 0);
    if (k < 64) {
      const S yk = read_lane(sv, k);
      return apply<Alg>(compose<Alg>(F, acc), yk);
    }
    acc = compose<Alg>(F, acc);
    base -= 64;
  }
}

// End of a workgroup: count it as finished; the last one resets the header
// for the next call on this workspace (see "Self-resetting workspace").
__device__ __forceinline__ void retire_block(unsigned *header, uint64_t *status, int64_t capacity,
                                             unsigned tag, int &s_last) {
  // every wave drains its outstanding memory operations first, so no status
  // read of this block can still be in flight when the last block resets
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(header + kHdrDone, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == gridDim.x - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  const bool wrap = (tag == 0xFFFFFFFFu);
  if (wrap)
    for (int64_t i = threadIdx.x; i < capacity; i += blockDim.x)
      __hip_atomic_store(status + i, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (threadIdx.x == 0) {
    __hip_atomic_store(header + kHdrCounter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(header + kHdrDone, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(header + kHdrEpoch, wrap ? 0u : tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------ chunk I/O
template <typename X, int K>
__device__ __forceinline__ void load_chunk(const X *row, int64_t t0, int64_t T, bool vec, X (&out)[K],
                                           const X &fill) {
  if (vec && t0 + K <= T) {
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
    for (int k = 0; k < K; ++k) out[k] = (t0 + k < T) ? row[t0 + k] : fill;
  }
}

template <typename X, int K>
__device__ __forceinline__ void store_chunk(X *row, int64_t t0, int64_t T, bool vec, const X (&v)[K]) {
  if (vec && t0 + K <= T) {
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

// ------------------------------------------------------------ the kernel
// TV  : the coefficient varies along time (LPV); otherwise one per row (LTI).
// REV : backward adjoint scan, nu[t] = A[t]^H (g[t] + nu[t+1]), run from the
//       end of the row towards its start; lambda[t] = g[t] + nu[t+1] is
//       grad_x, lambda[t] conj(y[t-1])^T the coefficient grad, nu[0] grad_zi.
template <class Alg, bool TV, bool REV>
__global__ __launch_bounds__(kThreads) void scan_kernel(ScanArgs<Alg> a) {
  using C = typename Alg::coef;      // compute types
  using S = typename Alg::state;
  using SC = typename Alg::s_coef;   // storage types
  using SS = typename Alg::s_state;
  using M = Map<Alg>;
  using Sh = Shape<Alg>;
  constexpr int K = Sh::K, R = Sh::R;

  __shared__ M s_wagg[kWaves];
  __shared__ S s_in;
  __shared__ unsigned s_id, s_tag;
  __shared__ int s_last;
  __shared__ typename Alg::acc_coef s_acc[kWaves];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid == 0) {
    s_id = __hip_atomic_fetch_add(a.header + kHdrCounter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_tag = __hip_atomic_load(a.header + kHdrEpoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  }
  __syncthreads();
  const int64_t id = s_id;
  const unsigned tag = s_tag;
  const int64_t qs = id / a.B;         // position in scan order
  const int64_t b = id - qs * a.B;
  const int64_t qf = REV ? a.tiles_per_row - 1 - qs : qs;  // position along time
  const int64_t T = a.T_len;
  const int64_t seg0 = qf * Sh::kTile + int64_t(w) * Sh::kWaveSeg;
  const bool vec = a.vec_ok != 0;

  const SS *xrow = reinterpret_cast<const SS *>(a.x) + b * T;
  const SC *crow = reinterpret_cast<const SC *>(a.coef) + b * a.coef_row_stride;
  const SS *yrow_in = reinterpret_cast<const SS *>(a.y) + b * T;
  const S zero_s = Alg::szero();
  // Steps past the end of the row load a zero coefficient and a zero input.
  // Forward they follow every valid step, so they only touch the aggregate of
  // the row's last tile, which nobody reads.  Backward they come first, where
  // the carry is zero anyway, and keep it zero.
  const SC zero_sc = Alg::s_czero();
  const SS zero_ss = Alg::s_szero();

  // ---- loads (all rounds issued up front)
  SS X[R][K];
  SC A[TV ? R : 1][TV ? K : 1];
  SS Y[REV ? R : 1][REV ? K : 1];
  SS Yfirst[REV ? R : 1];  // backward: y[t-1] for lane 0 of each round
  C a_row = Alg::load_c(zero_sc);
  if (!TV) a_row = Alg::load_c(crow[0]);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t t0 = seg0 + int64_t(r) * 64 * K + int64_t(lane) * K;
    load_chunk<SS, K>(xrow, t0, T, vec, X[r], zero_ss);
    if constexpr (TV) load_chunk<SC, K>(crow, t0, T, vec, A[r], zero_sc);
    if constexpr (REV) {
      load_chunk<SS, K>(yrow_in, t0, T, vec, Y[r], zero_ss);
      Yfirst[r] = zero_ss;
      if (lane == 0) {
        if (t0 == 0)
          Yfirst[r] = reinterpret_cast<const SS *>(a.zi)[b];
        else if (t0 - 1 < T)
          Yfirst[r] = yrow_in[t0 - 1];
      }
    }
  }
  auto coef_at = [&](int r, int k) -> C {
    if constexpr (TV) {
      const C v = Alg::load_c(A[r][k]);
      return REV ? Alg::adjoint(v) : v;
    } else {
      return REV ? Alg::adjoint(a_row) : a_row;
    }
  };

  // ---- pass 1: lane maps, wave scans, round chaining
  M Ex[R];
  M carry = map_identity<Alg>();
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    const int r = REV ? R - 1 - rr : rr;
    M m = map_identity<Alg>();
#pragma unroll
    for (int kk = 0; kk < K; ++kk) {
      const int k = REV ? K - 1 - kk : kk;
      const C c = coef_at(r, k);
      const S xv = Alg::load_s(X[r][k]);
      M e;
      e.A = c;
      e.x = REV ? Alg::affine(c, xv, zero_s) : xv;
      m = compose<Alg>(m, e);
    }
    // inclusive scan over lanes in scan order
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int src = REV ? lane + d : lane - d;
      M o = shfl_from(m, src);
      if (REV ? (lane + d < 64) : (lane >= d)) m = compose<Alg>(o, m);
    }
    M ex = shfl_from(m, REV ? lane + 1 : lane - 1);
    if (lane == (REV ? 63 : 0)) ex = map_identity<Alg>();
    const M tot = read_lane(m, REV ? 0 : 63);
    Ex[r] = compose<Alg>(carry, ex);
    carry = compose<Alg>(carry, tot);
  }

  // ---- block: wave aggregates in scan order
  if (lane == 0) s_wagg[w] = carry;
  __syncthreads();
  M wpre = map_identity<Alg>();
  M tagg = map_identity<Alg>();
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const int wi = REV ? kWaves - 1 - i : i;
    if (REV ? (wi > w) : (wi < w)) wpre = compose<Alg>(wpre, s_wagg[wi]);
    tagg = compose<Alg>(tagg, s_wagg[wi]);
  }

  // ---- look-back (wave 0)
  if (w == 0) {
    uint64_t *row_status = a.status + b * a.tiles_per_row * Sh::kStride;
    const S virt = REV ? zero_s : Alg::load_s(reinterpret_cast<const SS *>(a.zi)[b]);
    S yin;
    if (qs == 0) {
      yin = virt;
    } else {
      if (lane == 0) publish(row_status + qs * Sh::kStride + Sh::kIncWords, tagg, tag);
      yin = lookback<Alg>(row_status, qs, virt, lane, tag);
    }
    if (qs + 1 < a.tiles_per_row && lane == 0)
      publish(row_status + qs * Sh::kStride, apply<Alg>(tagg, yin), tag);
    if (lane == 0) s_in = yin;
  }
  __syncthreads();
  const S hw = apply<Alg>(wpre, s_in);

  // ---- pass 2
  if constexpr (!REV) {
    SS *yrow = reinterpret_cast<SS *>(a.out) + b * T;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t t0 = seg0 + int64_t(r) * 64 * K + int64_t(lane) * K;
      S h = apply<Alg>(Ex[r], hw);
      SS O[K];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        h = Alg::affine(coef_at(r, k), h, Alg::load_s(X[r][k]));
        O[k] = Alg::store_s(h);
      }
      store_chunk<SS, K>(yrow, t0, T, vec, O);
    }
  } else {
    SS *gxrow = a.out ? reinterpret_cast<SS *>(a.out) + b * T : nullptr;
    SC *gcrow = a.gcoef ? reinterpret_cast<SC *>(a.gcoef) + b * T : nullptr;
    typename Alg::acc_coef acc = Alg::acc_zero();
    const bool want_acc = a.partials != nullptr;
    // the rounds are walked from the end of the segment towards its start
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      const int r = R - 1 - rr;
      const int64_t t0 = seg0 + int64_t(r) * 64 * K + int64_t(lane) * K;
      // y[t-1] for each of this lane's steps: own registers, the previous
      // lane's last step, or (lane 0) the value loaded from memory
      SS yp0 = shfl_from(Y[r][K - 1], lane - 1);
      if (lane == 0) yp0 = Yfirst[r];
      S nu = apply<Alg>(Ex[r], hw);
      SS GX[K];
      SC GC[K];
#pragma unroll
      for (int kk = 0; kk < K; ++kk) {
        const int k = K - 1 - kk;
        const C c = coef_at(r, k);
        const S lam = Alg::sadd(Alg::load_s(X[r][k]), nu);
        GX[k] = Alg::store_s(lam);
        const S yprev = Alg::load_s(k == 0 ? yp0 : Y[r][k > 0 ? k - 1 : 0]);
        const C g = Alg::outer(lam, yprev);
        GC[k] = Alg::store_c(g);
        if (want_acc && t0 + k < T) acc = Alg::acc_add(acc, g);
        nu = Alg::affine(c, lam, zero_s);
        if (t0 + k == 0 && a.gzi) reinterpret_cast<SS *>(a.gzi)[b] = Alg::store_s(nu);
      }
      if (gxrow) store_chunk<SS, K>(gxrow, t0, T, vec, GX);
      if constexpr (TV) {
        if (gcrow) store_chunk<SC, K>(gcrow, t0, T, vec, GC);
      }
    }
    if (want_acc) {
      // deterministic block reduction of the per-tile coefficient gradient
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) acc = Alg::acc_sum(acc, shfl_from(acc, lane ^ d));
      if (lane == 0) s_acc[w] = acc;
      __syncthreads();
      if (tid == 0) {
        typename Alg::acc_coef sum = s_acc[0];
#pragma unroll
        for (int i = 1; i < kWaves; ++i) sum = Alg::acc_sum(sum, s_acc[i]);
        reinterpret_cast<typename Alg::acc_coef *>(a.partials)[b * a.tiles_per_row + qf] = sum;
      }
    }
  }
  retire_block(a.header, a.status, a.status_capacity, tag, s_last);
}

// ------------------------------------------------------------ helpers
// out[i] = sum_{j < count} partials[i*count + j], fixed order, one block per i.
template <class Alg>
__global__ __launch_bounds__(kThreads) void reduce_rows_kernel(const void *partials, int64_t count,
                                                                typename Alg::elem *out) {
  using AC = typename Alg::acc_coef;
  __shared__ AC s[kThreads];
  const AC *p = reinterpret_cast<const AC *>(partials) + blockIdx.x * count;
  AC acc = Alg::acc_zero();
  for (int64_t j = threadIdx.x; j < count; j += kThreads) acc = Alg::acc_sum(acc, p[j]);
  s[threadIdx.x] = acc;
  __syncthreads();
  for (int h = kThreads / 2; h > 0; h >>= 1) {
    if (threadIdx.x < h) s[threadIdx.x] = Alg::acc_sum(s[threadIdx.x], s[threadIdx.x + h]);
    __syncthreads();
  }
  if (threadIdx.x == 0)
    reinterpret_cast<typename Alg::s_coef *>(out)[blockIdx.x] = Alg::store_c(s[0]);
}

// out[t] = sum_b per_step[b, t]  (LPV coefficient shared across the batch).
template <class Alg>
__global__ __launch_bounds__(kThreads) void reduce_batch_kernel(const typename Alg::elem *per_step,
                                                                 int64_t B, int64_t T,
                                                                 typename Alg::elem *out) {
  using SC = typename Alg::s_coef;
  const SC *p = reinterpret_cast<const SC *>(per_step);
  for (int64_t t = blockIdx.x * int64_t(kThreads) + threadIdx.x; t < T;
       t += int64_t(gridDim.x) * kThreads) {
    typename Alg::acc_coef acc = Alg::acc_zero();
    for (int64_t b = 0; b < B; ++b) acc = Alg::acc_add(acc, Alg::load_c(p[b * T + t]));
    reinterpret_cast<SC *>(out)[t] = Alg::store_c(acc);
  }
}

}  // namespace phs
