// Achievable-bandwidth probe (measurement only, no counterpart in the
// reference): streaming kernels that move the same bytes as the scans, with
// no scan and no look-back, so that the bench can report how close a scan
// launch comes to a plain kernel of the same traffic and launch shape.
//
//   shape 0  the fp32 scalar scan's tile geometry: 8 waves of 64 lanes, a
//            lane holding 4 consecutive floats (one float4) per array in
//            each of four rounds (8192 elements per workgroup, one tile per
//            workgroup), every load issued before the first store
//   shape 1  one float4 per lane and array, 2048 elements per workgroup
//   shape 2  shape 0's grid with no memory access: launch and drain only
//
// out_j[i] = (j + 1) * sum_k in_k[i], so every input is read.
#include "phs_launch.hpp"

namespace phs {
namespace {

struct ProbeArgs {
  const float *in[3];
  float *out[2];
  int64_t n;
};

template <int NIN, int NOUT>
__global__ __launch_bounds__(512) void probe_tile_kernel(ProbeArgs a) {
  constexpr int kRounds = 4;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int64_t base = int64_t(blockIdx.x) * 8192 + w * 1024 + l * 4;
  float4 v[NIN][kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r)
#pragma unroll
    for (int k = 0; k < NIN; ++k) v[k][r] = *reinterpret_cast<const float4 *>(a.in[k] + base + r * 256);
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    float4 s = v[0][r];
#pragma unroll
    for (int k = 1; k < NIN; ++k) {
      s.x += v[k][r].x;
      s.y += v[k][r].y;
      s.z += v[k][r].z;
      s.w += v[k][r].w;
    }
#pragma unroll
    for (int j = 0; j < NOUT; ++j) {
      const float c = float(j + 1);
      *reinterpret_cast<float4 *>(a.out[j] + base + r * 256) = make_float4(c * s.x, c * s.y, c * s.z, c * s.w);
    }
  }
}

template <int NIN, int NOUT>
__global__ __launch_bounds__(512) void probe_flat_kernel(ProbeArgs a) {
  const int64_t i = (int64_t(blockIdx.x) * 512 + threadIdx.x) * 4;
  float4 s = reinterpret_cast<const float4 *>(a.in[0] + i)[0];
#pragma unroll
  for (int k = 1; k < NIN; ++k) {
    const float4 v = reinterpret_cast<const float4 *>(a.in[k] + i)[0];
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
#pragma unroll
  for (int j = 0; j < NOUT; ++j) {
    const float c = float(j + 1);
    reinterpret_cast<float4 *>(a.out[j] + i)[0] = make_float4(c * s.x, c * s.y, c * s.z, c * s.w);
  }
}

__global__ __launch_bounds__(512) void probe_empty_kernel(ProbeArgs a) {
  if (a.n < 0 && threadIdx.x == 0) a.out[0][0] = 0.f;  // never taken (n >= 0)
}

template <int NIN, int NOUT>
void launch_probe(int shape, const ProbeArgs &a, hipStream_t s) {
  if (shape == 0)
    phs::launch_kernel((probe_tile_kernel<NIN, NOUT>), dim3(unsigned(a.n / 8192)), dim3(512), 0, s, a);
  else
    phs::launch_kernel((probe_flat_kernel<NIN, NOUT>), dim3(unsigned(a.n / 2048)), dim3(512), 0, s, a);
}

}  // namespace
}  // namespace phs

extern "C" int phs_stream_probe(int shape, int n_in, int n_out, int64_t n, const void *const *in,
                                void *const *out, void *stream) {
  using namespace phs;
  if (shape < 0 || shape > 2 || n_in < 1 || n_in > 3 || n_out < 1 || n_out > 2 || n <= 0 || n % 8192 != 0 ||
      n / 8192 > (int64_t(1) << 30) || !in || !out)
    return PHS_ERR_INVALID;
  ProbeArgs a{};
  for (int k = 0; k < n_in; ++k) {
    if (!in[k] || (reinterpret_cast<uintptr_t>(in[k]) & 15u)) return PHS_ERR_INVALID;
    a.in[k] = static_cast<const float *>(in[k]);
  }
  for (int j = 0; j < n_out; ++j) {
    if (!out[j] || (reinterpret_cast<uintptr_t>(out[j]) & 15u)) return PHS_ERR_INVALID;
    a.out[j] = static_cast<float *>(out[j]);
  }
  a.n = n;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (shape == 2) {
    phs::launch_kernel(probe_empty_kernel, dim3(unsigned(n / 8192)), dim3(512), 0, s, a);
  } else {
    switch (n_in * 4 + n_out) {
      case 1 * 4 + 1: launch_probe<1, 1>(shape, a, s); break;
      case 2 * 4 + 1: launch_probe<2, 1>(shape, a, s); break;
      case 3 * 4 + 2: launch_probe<3, 2>(shape, a, s); break;
      case 3 * 4 + 1: launch_probe<3, 1>(shape, a, s); break;
      case 2 * 4 + 2: launch_probe<2, 2>(shape, a, s); break;
      case 1 * 4 + 2: launch_probe<1, 2>(shape, a, s); break;
      default: return PHS_ERR_INVALID;
    }
  }
  return hipGetLastError() == hipSuccess ? PHS_OK : PHS_ERR_LAUNCH;
}
