// Element algebra of the linear-recurrence scans.
//
// A step of `h[t] = A[t] h[t-1] + x[t]` is the affine map  h -> A h + x.
// Maps compose associatively:  (first p, then q) = (q.A p.A, q.A p.x + q.x),
// which is the operator the reference scans with Thrust
// (philtorch/csrc/lti_recur.cu:19-31 for the scalar case,
//  philtorch/csrc/recur2.cuh:7-21 for the 2x2 case).  Everything here is
// written for gfx950 wave64 code: values are moved between lanes as 32-bit
// words with ds_bpermute (`__shfl`) or v_readlane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace phs {

// ---------------------------------------------------------------- scalars
struct c64 {
  float re, im;
};
struct c128 {
  double re, im;
};

template <typename T>
struct Num;

template <>
struct Num<float> {
  static constexpr bool kComplex = false;
  using acc = double;
  static __device__ __forceinline__ float zero() { return 0.f; }
  static __device__ __forceinline__ float one() { return 1.f; }
};
template <>
struct Num<double> {
  static constexpr bool kComplex = false;
  using acc = double;
  static __device__ __forceinline__ double zero() { return 0.0; }
  static __device__ __forceinline__ double one() { return 1.0; }
};
template <>
struct Num<int64_t> {
  static constexpr bool kComplex = false;
  using acc = int64_t;
  static __device__ __forceinline__ int64_t zero() { return 0; }
  static __device__ __forceinline__ int64_t one() { return 1; }
};
template <>
struct Num<c64> {
  static constexpr bool kComplex = true;
  using acc = c128;
  static __device__ __forceinline__ c64 zero() { return {0.f, 0.f}; }
  static __device__ __forceinline__ c64 one() { return {1.f, 0.f}; }
};
template <>
struct Num<c128> {
  static constexpr bool kComplex = true;
  using acc = c128;
  static __device__ __forceinline__ c128 zero() { return {0.0, 0.0}; }
  static __device__ __forceinline__ c128 one() { return {1.0, 0.0}; }
};

// real arithmetic
__device__ __forceinline__ float mul(float a, float b) { return a * b; }
__device__ __forceinline__ double mul(double a, double b) { return a * b; }
__device__ __forceinline__ int64_t mul(int64_t a, int64_t b) { return a * b; }
__device__ __forceinline__ float add(float a, float b) { return a + b; }
__device__ __forceinline__ double add(double a, double b) { return a + b; }
__device__ __forceinline__ int64_t add(int64_t a, int64_t b) { return a + b; }
// a*b + c
__device__ __forceinline__ float mad(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double mad(double a, double b, double c) { return __builtin_fma(a, b, c); }
__device__ __forceinline__ int64_t mad(int64_t a, int64_t b, int64_t c) { return a * b + c; }
__device__ __forceinline__ float cj(float a) { return a; }
__device__ __forceinline__ double cj(double a) { return a; }
__device__ __forceinline__ int64_t cj(int64_t a) { return a; }

// complex arithmetic
template <typename C, typename R>
__device__ __forceinline__ C cmul(C a, C b) {
  C r;
  r.re = mad(a.re, b.re, -(a.im * b.im));
  r.im = mad(a.re, b.im, a.im * b.re);
  return r;
}
template <typename C>
__device__ __forceinline__ C cmad(C a, C b, C c) {
  C r;
  r.re = mad(a.re, b.re, mad(-a.im, b.im, c.re));
  r.im = mad(a.re, b.im, mad(a.im, b.re, c.im));
  return r;
}
__device__ __forceinline__ c64 mul(c64 a, c64 b) { return cmul<c64, float>(a, b); }
__device__ __forceinline__ c128 mul(c128 a, c128 b) { return cmul<c128, double>(a, b); }
__device__ __forceinline__ c64 add(c64 a, c64 b) { return {a.re + b.re, a.im + b.im}; }
__device__ __forceinline__ c128 add(c128 a, c128 b) { return {a.re + b.re, a.im + b.im}; }
__device__ __forceinline__ c64 mad(c64 a, c64 b, c64 c) { return cmad(a, b, c); }
__device__ __forceinline__ c128 mad(c128 a, c128 b, c128 c) { return cmad(a, b, c); }
__device__ __forceinline__ c64 cj(c64 a) { return {a.re, -a.im}; }
__device__ __forceinline__ c128 cj(c128 a) { return {a.re, -a.im}; }

// widening into the reduction accumulator type
__device__ __forceinline__ double widen(float v) { return (double)v; }
__device__ __forceinline__ double widen(double v) { return v; }
__device__ __forceinline__ int64_t widen(int64_t v) { return v; }
__device__ __forceinline__ c128 widen(c64 v) { return {(double)v.re, (double)v.im}; }
__device__ __forceinline__ c128 widen(c128 v) { return v; }
__device__ __forceinline__ void narrow(double v, float &o) { o = (float)v; }
__device__ __forceinline__ void narrow(double v, double &o) { o = v; }
__device__ __forceinline__ void narrow(int64_t v, int64_t &o) { o = v; }
__device__ __forceinline__ void narrow(c128 v, c64 &o) { o = {(float)v.re, (float)v.im}; }
__device__ __forceinline__ void narrow(c128 v, c128 &o) { o = v; }

// ---------------------------------------------------------------- 2x2 blocks
template <typename T>
struct Mat2 {
  T m00, m01, m10, m11;
};
template <typename T>
struct Vec2 {
  T v0, v1;
};

// ---------------------------------------------------------------- algebras
// Storage vs compute precision: data move in the caller's dtype, but every
// scan operation (lane folds, map compositions, look-back payloads and
// reductions) runs in the wide type below.  The path is bandwidth-bound, so
// fp64 arithmetic costs no throughput, and it keeps the parallel
// reassociation far inside the fp32 parity bar even for non-normal 2x2
// sections with poles near the unit circle.
template <typename T>
struct Wide {
  using type = T;
};
template <>
struct Wide<float> {
  using type = double;
};
template <>
struct Wide<c64> {
  using type = c128;
};

template <typename T>
__device__ __forceinline__ typename Wide<T>::type up(T v) {
  return widen(v);
}
template <typename T>
__device__ __forceinline__ T down(typename Wide<T>::type v) {
  T o;
  narrow(v, o);
  return o;
}

// Scalar first-order scan: coefficient and state are both one scalar.
template <typename T>
struct Scalar {
  using elem = T;                       // storage scalar
  using ct = typename Wide<T>::type;    // compute scalar
  using s_coef = T;                     // coefficient as stored
  using s_state = T;                    // state as stored
  using coef = ct;
  using state = ct;
  using acc_coef = ct;
  static constexpr int kCoefElems = 1;
  static constexpr int kStateElems = 1;
  // Real scans: one 16-byte vector per lane, array and round, in four
  // rounds (fp32: 4 steps x 4 rounds, a 8192-step tile).  Folding a round as
  // soon as its vectors arrive, with four rounds in flight, beat two rounds
  // of two vectors (C1 step 33.90 -> 32.37 us, same-box A/B).
  // LTI scans load no coefficients: complex lanes then carry twice the steps
  // in the registers the coefficients would take
  static constexpr int kVecsPerLane = Num<T>::kComplex ? 2 : 1;
  static constexpr int kVecsPerLaneLTI = Num<T>::kComplex ? 4 : 1;
  static constexpr int kRounds = Num<T>::kComplex ? 2 : 4;

  // Real scans: 8 data waves that also do the look-back, with a floor of 4
  // waves per SIMD (at most 128 VGPRs): two tiles resident per CU.  Complex
  // scans: 3 data waves plus a look-back wave, so the look-back's registers
  // do not add to the data path's (workgroups stay whole multiples of 4
  // waves, which the wave-slot allocation favours).
  static constexpr bool kLookbackWave = Num<T>::kComplex;
  static constexpr int kWavesPerBlock = Num<T>::kComplex ? 3 : 8;
  static constexpr int kMinWavesPerEU = Num<T>::kComplex ? 1 : 4;
  // tiles in the first look-back window (later windows hold 64): scalar
  // status entries are short and the nearest inclusive predecessor is usually
  // among the last 8 tiles (C5 fp32: 8 tiles 134, 16 tiles 125, 64 tiles 128
  // GSamples/s)
  static constexpr int kLookFirst = 8;

  static __device__ __forceinline__ coef load_c(s_coef v) { return up(v); }
  static __device__ __forceinline__ state load_s(s_state v) { return up(v); }
  static __device__ __forceinline__ s_coef store_c(coef v) { return down<T>(v); }
  static __device__ __forceinline__ s_state store_s(state v) { return down<T>(v); }
  static __device__ __forceinline__ s_coef s_czero() { return Num<T>::zero(); }
  static __device__ __forceinline__ s_state s_szero() { return Num<T>::zero(); }

  // steps of pass 2 run in storage precision from a wide entry state
  static __device__ __forceinline__ s_state s_affine(s_coef A, s_state h, s_state x) { return mad(A, h, x); }
  static __device__ __forceinline__ s_coef s_cmul(s_coef q, s_coef p) { return mul(q, p); }
  static __device__ __forceinline__ s_state s_add(s_state a, s_state b) { return add(a, b); }
  static __device__ __forceinline__ s_coef s_adjoint(s_coef A) { return cj(A); }
  static __device__ __forceinline__ s_coef s_outer(s_state lam, s_state y) { return mul(lam, cj(y)); }

  static __device__ __forceinline__ coef cone() { return Num<ct>::one(); }
  static __device__ __forceinline__ state szero() { return Num<ct>::zero(); }
  // q * p  (apply p first)
  static __device__ __forceinline__ coef cmul(coef q, coef p) { return mul(q, p); }
  // A h + x
  static __device__ __forceinline__ state affine(coef A, state h, state x) { return mad(A, h, x); }
  static __device__ __forceinline__ state sadd(state a, state b) { return add(a, b); }
  // A^H (conjugate transpose)
  static __device__ __forceinline__ coef adjoint(coef A) { return cj(A); }
  // lambda conj(y)^T : the per-step gradient of the coefficient
  static __device__ __forceinline__ coef outer(state lam, state y) { return mul(lam, cj(y)); }
  static __device__ __forceinline__ acc_coef acc_zero() { return Num<ct>::zero(); }
  static __device__ __forceinline__ acc_coef acc_add(acc_coef s, coef v) { return add(s, v); }
  static __device__ __forceinline__ acc_coef acc_sum(acc_coef a, acc_coef b) { return add(a, b); }
};

// 2x2 state-space recursion (biquad sections): coefficient Mat2, state Vec2.
template <typename T>
struct Block2 {
  using elem = T;
  using ct = typename Wide<T>::type;
  using s_coef = Mat2<T>;
  using s_state = Vec2<T>;
  using coef = Mat2<ct>;
  using state = Vec2<ct>;
  using acc_coef = Mat2<ct>;
  static constexpr int kCoefElems = 4;
  static constexpr int kStateElems = 2;
  static constexpr int kVecsPerLane = 2;
  static constexpr int kVecsPerLaneLTI = 4;  // LTI: no per-step coefficients to hold (see Scalar)
  static constexpr int kRounds = 2;
  // 3 data waves plus a look-back wave (see Scalar); real 2x2 scans keep a
  // floor of 3 waves per SIMD (at most 168 VGPRs), complex ones would spill
  // heavily under it
  static constexpr bool kLookbackWave = true;
  static constexpr int kWavesPerBlock = 3;
  static constexpr int kMinWavesPerEU = Num<T>::kComplex ? 1 : 3;
  // a full first look-back window: a short one costs 2x2 scans a second poll
  // too often (C3: 8 tiles 40.7, 16 tiles 38.8, 64 tiles 45.5 GSamples/s)
  static constexpr int kLookFirst = 64;

  static __device__ __forceinline__ coef load_c(s_coef v) {
    return {up(v.m00), up(v.m01), up(v.m10), up(v.m11)};
  }
  static __device__ __forceinline__ state load_s(s_state v) { return {up(v.v0), up(v.v1)}; }
  static __device__ __forceinline__ s_coef store_c(coef v) {
    return {down<T>(v.m00), down<T>(v.m01), down<T>(v.m10), down<T>(v.m11)};
  }
  static __device__ __forceinline__ s_state store_s(state v) { return {down<T>(v.v0), down<T>(v.v1)}; }
  static __device__ __forceinline__ s_coef s_czero() {
    return {Num<T>::zero(), Num<T>::zero(), Num<T>::zero(), Num<T>::zero()};
  }
  static __device__ __forceinline__ s_state s_szero() { return {Num<T>::zero(), Num<T>::zero()}; }

  static __device__ __forceinline__ s_state s_affine(s_coef A, s_state h, s_state x) {
    return {mad(A.m00, h.v0, mad(A.m01, h.v1, x.v0)), mad(A.m10, h.v0, mad(A.m11, h.v1, x.v1))};
  }
  static __device__ __forceinline__ s_state s_add(s_state a, s_state b) {
    return {add(a.v0, b.v0), add(a.v1, b.v1)};
  }
  static __device__ __forceinline__ s_coef s_cmul(s_coef q, s_coef p) {
    return {mad(q.m00, p.m00, mul(q.m01, p.m10)), mad(q.m00, p.m01, mul(q.m01, p.m11)),
            mad(q.m10, p.m00, mul(q.m11, p.m10)), mad(q.m10, p.m01, mul(q.m11, p.m11))};
  }
  static __device__ __forceinline__ s_coef s_adjoint(s_coef A) {
    return {cj(A.m00), cj(A.m10), cj(A.m01), cj(A.m11)};
  }
  static __device__ __forceinline__ s_coef s_outer(s_state lam, s_state y) {
    T y0 = cj(y.v0), y1 = cj(y.v1);
    return {mul(lam.v0, y0), mul(lam.v0, y1), mul(lam.v1, y0), mul(lam.v1, y1)};
  }

  static __device__ __forceinline__ coef cone() {
    return {Num<ct>::one(), Num<ct>::zero(), Num<ct>::zero(), Num<ct>::one()};
  }
  static __device__ __forceinline__ state szero() { return {Num<ct>::zero(), Num<ct>::zero()}; }
  static __device__ __forceinline__ coef cmul(coef q, coef p) {
    coef r;
    r.m00 = mad(q.m00, p.m00, mul(q.m01, p.m10));
    r.m01 = mad(q.m00, p.m01, mul(q.m01, p.m11));
    r.m10 = mad(q.m10, p.m00, mul(q.m11, p.m10));
    r.m11 = mad(q.m10, p.m01, mul(q.m11, p.m11));
    return r;
  }
  static __device__ __forceinline__ state affine(coef A, state h, state x) {
    state r;
    r.v0 = mad(A.m00, h.v0, mad(A.m01, h.v1, x.v0));
    r.v1 = mad(A.m10, h.v0, mad(A.m11, h.v1, x.v1));
    return r;
  }
  static __device__ __forceinline__ state sadd(state a, state b) {
    return {add(a.v0, b.v0), add(a.v1, b.v1)};
  }
  static __device__ __forceinline__ coef adjoint(coef A) {
    return {cj(A.m00), cj(A.m10), cj(A.m01), cj(A.m11)};
  }
  static __device__ __forceinline__ coef outer(state lam, state y) {
    ct y0 = cj(y.v0), y1 = cj(y.v1);
    return {mul(lam.v0, y0), mul(lam.v0, y1), mul(lam.v1, y0), mul(lam.v1, y1)};
  }
  static __device__ __forceinline__ acc_coef acc_zero() {
    return {Num<ct>::zero(), Num<ct>::zero(), Num<ct>::zero(), Num<ct>::zero()};
  }
  static __device__ __forceinline__ acc_coef acc_add(acc_coef s, coef v) {
    return {add(s.m00, v.m00), add(s.m01, v.m01), add(s.m10, v.m10), add(s.m11, v.m11)};
  }
  static __device__ __forceinline__ acc_coef acc_sum(acc_coef a, acc_coef b) {
    return {add(a.m00, b.m00), add(a.m01, b.m01), add(a.m10, b.m10), add(a.m11, b.m11)};
  }
};

// M x M state-space recursion for small orders (M = 3, 4): coefficient MatN
// (row-major, as torch stores [..., M, M]), state VecN.  The generic
// counterpart of Block2, which stays hand-unrolled for the biquad hot path.
template <typename T, int M>
struct MatN {
  T m[M * M];
};
template <typename T, int M>
struct VecN {
  T v[M];
};

template <typename T, int M>
struct BlockN {
  using elem = T;
  using ct = typename Wide<T>::type;
  using s_coef = MatN<T, M>;
  using s_state = VecN<T, M>;
  using coef = MatN<ct, M>;
  using state = VecN<ct, M>;
  using acc_coef = MatN<ct, M>;
  static constexpr int kCoefElems = M * M;
  static constexpr int kStateElems = M;
  static constexpr int kVecsPerLane = 1;
  static constexpr int kVecsPerLaneLTI = 1;
  static constexpr int kRounds = 2;
  // 3 data waves plus a look-back wave, as Block2; no register floor (the
  // maps are large and complex orders would spill under one)
  static constexpr bool kLookbackWave = true;
  static constexpr int kWavesPerBlock = 3;
  static constexpr int kMinWavesPerEU = 1;
  static constexpr int kLookFirst = 64;  // as Block2

  template <typename D, typename S, int N>
  static __device__ __forceinline__ void conv_up(D (&d)[N], const S (&s)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) d[i] = up(s[i]);
  }
  template <typename D, typename S, int N>
  static __device__ __forceinline__ void conv_down(D (&d)[N], const S (&s)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) d[i] = down<T>(s[i]);
  }
  template <typename U>
  static __device__ __forceinline__ MatN<U, M> mat_zero() {
    MatN<U, M> r;
#pragma unroll
    for (int i = 0; i < M * M; ++i) r.m[i] = Num<U>::zero();
    return r;
  }
  template <typename U>
  static __device__ __forceinline__ VecN<U, M> vec_zero() {
    VecN<U, M> r;
#pragma unroll
    for (int i = 0; i < M; ++i) r.v[i] = Num<U>::zero();
    return r;
  }
  // q p (apply p first)
  template <typename U>
  static __device__ __forceinline__ MatN<U, M> mat_mul(const MatN<U, M> &q, const MatN<U, M> &p) {
    MatN<U, M> r;
#pragma unroll
    for (int i = 0; i < M; ++i)
#pragma unroll
      for (int j = 0; j < M; ++j) {
        U acc = mul(q.m[i * M + M - 1], p.m[(M - 1) * M + j]);
#pragma unroll
        for (int k = M - 2; k >= 0; --k) acc = mad(q.m[i * M + k], p.m[k * M + j], acc);
        r.m[i * M + j] = acc;
      }
    return r;
  }
  // A h + x
  template <typename U>
  static __device__ __forceinline__ VecN<U, M> mat_affine(const MatN<U, M> &A, const VecN<U, M> &h,
                                                         const VecN<U, M> &x) {
    VecN<U, M> r;
#pragma unroll
    for (int i = 0; i < M; ++i) {
      U acc = x.v[i];
#pragma unroll
      for (int k = M - 1; k >= 0; --k) acc = mad(A.m[i * M + k], h.v[k], acc);
      r.v[i] = acc;
    }
    return r;
  }
  template <typename U>
  static __device__ __forceinline__ VecN<U, M> vec_add(const VecN<U, M> &a, const VecN<U, M> &b) {
    VecN<U, M> r;
#pragma unroll
    for (int i = 0; i < M; ++i) r.v[i] = add(a.v[i], b.v[i]);
    return r;
  }
  template <typename U>
  static __device__ __forceinline__ MatN<U, M> mat_adjoint(const MatN<U, M> &A) {
    MatN<U, M> r;
#pragma unroll
    for (int i = 0; i < M; ++i)
#pragma unroll
      for (int j = 0; j < M; ++j) r.m[i * M + j] = cj(A.m[j * M + i]);
    return r;
  }
  // lam conj(y)^T
  template <typename U>
  static __device__ __forceinline__ MatN<U, M> vec_outer(const VecN<U, M> &lam, const VecN<U, M> &y) {
    MatN<U, M> r;
#pragma unroll
    for (int i = 0; i < M; ++i)
#pragma unroll
      for (int j = 0; j < M; ++j) r.m[i * M + j] = mul(lam.v[i], cj(y.v[j]));
    return r;
  }

  static __device__ __forceinline__ coef load_c(const s_coef &v) {
    coef r;
    conv_up(r.m, v.m);
    return r;
  }
  static __device__ __forceinline__ state load_s(const s_state &v) {
    state r;
    conv_up(r.v, v.v);
    return r;
  }
  static __device__ __forceinline__ s_coef store_c(const coef &v) {
    s_coef r;
    conv_down(r.m, v.m);
    return r;
  }
  static __device__ __forceinline__ s_state store_s(const state &v) {
    s_state r;
    conv_down(r.v, v.v);
    return r;
  }
  static __device__ __forceinline__ s_coef s_czero() { return mat_zero<T>(); }
  static __device__ __forceinline__ s_state s_szero() { return vec_zero<T>(); }
  static __device__ __forceinline__ s_state s_affine(const s_coef &A, const s_state &h, const s_state &x) {
    return mat_affine<T>(A, h, x);
  }
  static __device__ __forceinline__ s_state s_add(const s_state &a, const s_state &b) { return vec_add<T>(a, b); }
  static __device__ __forceinline__ s_coef s_cmul(const s_coef &q, const s_coef &p) { return mat_mul<T>(q, p); }
  static __device__ __forceinline__ s_coef s_adjoint(const s_coef &A) { return mat_adjoint<T>(A); }
  static __device__ __forceinline__ s_coef s_outer(const s_state &lam, const s_state &y) {
    return vec_outer<T>(lam, y);
  }

  static __device__ __forceinline__ coef cone() {
    coef r = mat_zero<ct>();
#pragma unroll
    for (int i = 0; i < M; ++i) r.m[i * M + i] = Num<ct>::one();
    return r;
  }
  static __device__ __forceinline__ state szero() { return vec_zero<ct>(); }
  static __device__ __forceinline__ coef cmul(const coef &q, const coef &p) { return mat_mul<ct>(q, p); }
  static __device__ __forceinline__ state affine(const coef &A, const state &h, const state &x) {
    return mat_affine<ct>(A, h, x);
  }
  static __device__ __forceinline__ state sadd(const state &a, const state &b) { return vec_add<ct>(a, b); }
  static __device__ __forceinline__ coef adjoint(const coef &A) { return mat_adjoint<ct>(A); }
  static __device__ __forceinline__ coef outer(const state &lam, const state &y) { return vec_outer<ct>(lam, y); }
  static __device__ __forceinline__ acc_coef acc_zero() { return mat_zero<ct>(); }
  static __device__ __forceinline__ acc_coef acc_add(const acc_coef &s, const coef &v) {
    acc_coef r;
#pragma unroll
    for (int i = 0; i < M * M; ++i) r.m[i] = add(s.m[i], v.m[i]);
    return r;
  }
  static __device__ __forceinline__ acc_coef acc_sum(const acc_coef &a, const acc_coef &b) { return acc_add(a, b); }
};

// Affine map h -> A h + x.
template <class Alg>
struct Map {
  typename Alg::coef A;
  typename Alg::state x;
};

// The same map in storage precision (a lane's few steps are folded in it).
template <class Alg>
struct SMap {
  typename Alg::s_coef A;
  typename Alg::s_state x;
};

template <class Alg>
__device__ __forceinline__ Map<Alg> map_identity() {
  return {Alg::cone(), Alg::szero()};
}
// first p, then q
template <class Alg>
__device__ __forceinline__ Map<Alg> compose(const Map<Alg> &p, const Map<Alg> &q) {
  return {Alg::cmul(q.A, p.A), Alg::affine(q.A, p.x, q.x)};
}
template <class Alg>
__device__ __forceinline__ typename Alg::state apply(const Map<Alg> &m, const typename Alg::state &h) {
  return Alg::affine(m.A, h, m.x);
}

// ---------------------------------------------------------------- lane moves
template <typename X>
__device__ __forceinline__ X shfl_from(const X &v, int src) {
  static_assert(sizeof(X) % 4 == 0, "32-bit granular types only");
  constexpr int n = sizeof(X) / 4;
  union {
    X x;
    int w[n];
  } in, out;
  in.x = v;
#pragma unroll
  for (int i = 0; i < n; ++i) out.w[i] = __shfl(in.w[i], src, 64);
  return out.x;
}

// DPP lane move of every 32-bit word of `v` (gfx9 DPP control `CTRL`,
// rows enabled by `ROW_MASK`).  Lanes without a source, or in disabled rows,
// keep their own value.
template <int CTRL, int ROW_MASK, typename X>
__device__ __forceinline__ X dpp_move(const X &v) {
  constexpr int n = sizeof(X) / 4;
  union {
    X x;
    int w[n];
  } in, out;
  in.x = v;
#pragma unroll
  for (int i = 0; i < n; ++i) out.w[i] = __builtin_amdgcn_update_dpp(in.w[i], in.w[i], CTRL, ROW_MASK, 0xF, false);
  return out.x;
}

constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;
constexpr int kDppWaveShr1 = 0x138;

// Inclusive wave64 scan of `v` under the associative, non-commutative `op`
// (op(earlier, later)), lane 0 first: four row_shr steps inside each
// 16-lane row, then row_bcast:15 and row_bcast:31 across rows.
template <typename X, typename Op>
__device__ __forceinline__ X wave_scan_incl(X v, int lane, Op op) {
  const int r = lane & 15;
  X o;
  o = dpp_move<kDppRowShr1, 0xF>(v);
  if (r >= 1) v = op(o, v);
  o = dpp_move<kDppRowShr2, 0xF>(v);
  if (r >= 2) v = op(o, v);
  o = dpp_move<kDppRowShr4, 0xF>(v);
  if (r >= 4) v = op(o, v);
  o = dpp_move<kDppRowShr8, 0xF>(v);
  if (r >= 8) v = op(o, v);
  o = dpp_move<kDppRowBcast15, 0xA>(v);
  if (lane & 16) v = op(o, v);
  o = dpp_move<kDppRowBcast31, 0xC>(v);
  if (lane >= 32) v = op(o, v);
  return v;
}

// Value of the previous lane (lane 0 gets `first`).
template <typename X>
__device__ __forceinline__ X wave_shift_up(const X &v, int lane, const X &first) {
  X o = dpp_move<kDppWaveShr1, 0xF>(v);
  return lane == 0 ? first : o;
}

// Value of `v` held by lane `lane` (must be wave-uniform); result is uniform.
template <typename X>
__device__ __forceinline__ X read_lane(const X &v, int lane) {
  constexpr int n = sizeof(X) / 4;
  union {
    X x;
    int w[n];
  } in, out;
  in.x = v;
#pragma unroll
  for (int i = 0; i < n; ++i) out.w[i] = __builtin_amdgcn_readlane(in.w[i], lane);
  return out.x;
}

}  // namespace phs
