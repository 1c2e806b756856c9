// Measured ceilings for the roofline report (no reference counterpart).
//
// The published peaks (2.5 PFLOP/s dense fp16 / bf16 MFMA, 8 TB/s HBM) are not
// reachable figures on this part: the MFMA rate under load depends on the
// operand data (the clock drops with the switching activity of the operands),
// and one kernel streaming a few hundred MB from HBM tops out well below 8
// TB/s.  These two kernels measure what the hardware delivers for exactly the
// work the fused kernels do, so a kernel's time can be read against both the
// published peak and the measured ceiling:
//
//   kans_mfma_ceiling: back-to-back v_mfma_f32_32x32x16_{f16,bf16} on operand
//     fragments supplied by the caller (sampled from a layer's real basis
//     values and weights), at the fused block kernel's occupancy (8 waves of
//     8 accumulator tiles per CU, two waves per SIMD), nothing else issued;
//   kans_stream_ceiling: a read-only stream over a device buffer, 16 waves per
//     CU, four 16-byte loads per lane in flight (the best streaming shape
//     measured on this part), nothing else done with the data; timed with
//     plain and with non-temporal loads, the faster one reported (a buffer
//     larger than the MALL streams faster non-temporal, a smaller one re-read
//     by every launch partly hits the MALL with plain loads).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "kans_api_internal.h"

using namespace kans;

namespace {

constexpr int kCeilFrags = 16;  // operand fragments per matrix side

template <typename T> struct CeilMfma;
template <> struct CeilMfma<_Float16> {
  typedef half8 frag;
  static __device__ __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct CeilMfma<__bf16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

// Each wave holds 4 A and 8 B fragments (picked by its index from the 16 of
// each side) and runs `iters` x 32 MFMAs into 8 accumulator tiles: A fragment
// s feeds 8 consecutive MFMAs against rotating B fragments, as in the fused
// kernel's slot step.
template <typename T>
__global__ void __launch_bounds__(512) k_mfma_ceiling(const uint4* __restrict__ A, const uint4* __restrict__ Bf,
                                                      int iters, float* __restrict__ out) {
  typedef typename CeilMfma<T>::frag frag;
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 8 + (threadIdx.x >> 6);
  frag a[4], b[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint4 u = A[((w + 5 * i) % kCeilFrags) * 64 + lane];
    a[i] = *reinterpret_cast<frag*>(&u);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint4 u = Bf[((3 * w + i) % kCeilFrags) * 64 + lane];
    b[i] = *reinterpret_cast<frag*>(&u);
  }
  floatx16 acc[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[nb][r] = 0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) acc[nb] = CeilMfma<T>::mma(a[s], b[(nb + s) & 7], acc[nb]);
  }
  float sum = 0.0f;
#pragma unroll
  for (int nb = 0; nb < 8; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) sum += acc[nb][r];
  out[(long)w * 64 + lane] = sum;  // keeps every MFMA live
}

// Wave w reads the contiguous range [w * per_wave, (w + 1) * per_wave) of
// 16-byte words, 4 KB per iteration; the xor of everything it read goes to
// out[w] so no load is dead.  NT: non-temporal loads.
template <bool NT>
__global__ void __launch_bounds__(256) k_stream_ceiling(const uint4* __restrict__ p, long per_wave, long n,
                                                        unsigned* __restrict__ out) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const long w = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const long lo = w * per_wave, hi = lo + per_wave < n ? lo + per_wave : n;
  unsigned x = 0u;
  for (long i = lo; i < hi; i += 256) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long j = i + u * 64 + lane;
      if (j < hi) {
        if constexpr (NT) {
          const u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + j));
          v[u] = make_uint4(t.x, t.y, t.z, t.w);
        } else {
          v[u] = p[j];
        }
      } else {
        v[u] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  x ^= __shfl_xor(x, 1);
  if (lane == 0) out[w] = x;
}

int cu_count() {
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 256;
  return prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
}

// median of `reps` timed launches of `go` (after one untimed launch)
template <typename F>
int time_median(F go, int reps, float* ms) {
  hipStream_t st = kans_default_stream();
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0));
  HIP_TRY(hipEventCreate(&e1));
  std::vector<float> t;
  int rc = 0;
  for (int r = 0; r <= reps && rc == 0; ++r) {
    if (hipEventRecord(e0, st) != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "event record failed");
    go(st);
    if (hipGetLastError() != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "ceiling kernel launch failed");
    if (rc == 0 && (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess))
      rc = kans_fail(KANS_ERR_HIP, "event wait failed");
    float v = 0.0f;
    if (rc == 0 && hipEventElapsedTime(&v, e0, e1) != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "event time failed");
    if (rc == 0 && r > 0) t.push_back(v);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (rc) return rc;
  std::sort(t.begin(), t.end());
  *ms = t[t.size() / 2];
  return 0;
}

}  // namespace

int kans_mfma_ceiling(int dtype, const void* a_frags, const void* b_frags, int iters, double* tflops) {
  if (!a_frags || !b_frags || !tflops || iters <= 0 || (dtype != DT_F16 && dtype != DT_BF16))
    return kans_fail(KANS_ERR_ARG, "mfma ceiling: bad argument");
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  const size_t fb = (size_t)kCeilFrags * 64 * 16;
  DevBuf A, B, out;
  const int wgs = cu_count();
  if ((rc = A.reserve(fb)) || (rc = B.reserve(fb)) || (rc = out.reserve((size_t)wgs * 512 * sizeof(float)))) return rc;
  HIP_TRY(hipMemcpy(A.p, a_frags, fb, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(B.p, b_frags, fb, hipMemcpyHostToDevice));
  float ms = 0.0f;
  rc = time_median(
      [&](hipStream_t st) {
        if (dtype == DT_F16)
          hipLaunchKernelGGL(k_mfma_ceiling<_Float16>, dim3(wgs), dim3(512), 0, st, (const uint4*)A.p,
                             (const uint4*)B.p, iters, (float*)out.p);
        else
          hipLaunchKernelGGL(k_mfma_ceiling<__bf16>, dim3(wgs), dim3(512), 0, st, (const uint4*)A.p,
                             (const uint4*)B.p, iters, (float*)out.p);
      },
      5, &ms);
  if (rc) return rc;
  const double flops = (double)wgs * 8 * iters * 32 * (2.0 * 32 * 32 * 16);
  *tflops = flops / ((double)ms * 1e-3) / 1e12;
  return 0;
}

int kans_stream_ceiling(const void* buf, size_t bytes, double* gb_per_s) {
  if (!buf || !gb_per_s || bytes < 16 || ((uintptr_t)buf & 15)) return kans_fail(KANS_ERR_ARG, "stream ceiling: bad argument");
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  const long n = (long)(bytes / 16);
  const long waves = (long)cu_count() * 16;
  const long per_wave = (n + waves - 1) / waves;
  DevBuf out;
  if ((rc = out.reserve((size_t)waves * sizeof(unsigned)))) return rc;
  float ms_plain = 0.0f, ms_nt = 0.0f;
  rc = time_median(
      [&](hipStream_t st) {
        hipLaunchKernelGGL(k_stream_ceiling<false>, dim3((unsigned)(waves / 4)), dim3(256), 0, st,
                           (const uint4*)buf, per_wave, n, (unsigned*)out.p);
      },
      9, &ms_plain);
  if (rc) return rc;
  rc = time_median(
      [&](hipStream_t st) {
        hipLaunchKernelGGL(k_stream_ceiling<true>, dim3((unsigned)(waves / 4)), dim3(256), 0, st,
                           (const uint4*)buf, per_wave, n, (unsigned*)out.p);
      },
      9, &ms_nt);
  if (rc) return rc;
  *gb_per_s = (double)(n * 16) / ((double)std::min(ms_plain, ms_nt) * 1e-3) / 1e9;
  return 0;
}
