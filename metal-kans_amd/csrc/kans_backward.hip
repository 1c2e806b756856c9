// Fused Chebyshev KAN layer backward for gfx950 (fp32), without materialising
// the basis tensor Phi.
//
// Reference: metal_kan_cheby_backward_fused (metal_kan_bridge.mm:4532-4632),
// kernels fused_backward_cheby_dW / fused_backward_cheby_dX
// (fused_kan.metal:2053-2163), and the unfused metal_kan_cheby_backward
// (metal_kan_bridge.mm:2715-2850: Phi in a scratch buffer, MPS GEMMs), which
// computes the same quantities.  For y = bias + SiLU(x) W_base^T + Phi(x) W^T
// and an upstream gradient dY:
//
//   dW[o, i*K+k]  = sum_b dY[b,o] T_k(clamp x[b,i])
//   dW_base[o, i] = sum_b dY[b,o] SiLU(x[b,i])
//   dbias[o]      = sum_b dY[b,o]
//   dX[b, i]      = sum_k (dY W)[b, i*K+k] T'_k(x[b,i]) + (dY W_base)[b,i] SiLU'(x[b,i])
//
// with T'_k taken as 0 where the raw input lies outside [-1, 1] (the clamp is
// flat there).  The reference dW kernel keeps at most 16 coefficients in
// registers; here K goes up to kMaxK.
//
// Both kernels contract over one axis against an operand with KP = K +
// has_base "slots" per feature (slot 0 = SiLU when has_base):
//   * k_cheby_bwd_dw: output tile 64 o x 16 features x KP slots, contraction
//     over the batch.  Per chunk of 16 rows the workgroup evaluates the slots
//     of its 16 x 16 (row, feature) pairs once into LDS; lane o of wave w
//     accumulates features 4w..4w+3 (the slot reads are LDS broadcasts).  The
//     workgroups of the first feature tile also reduce dbias.
//   * k_cheby_bwd_dx: output tile 64 rows x 16 features, contraction over
//     D_out in chunks of 16 against W / W_base tiles in LDS; the epilogue
//     multiplies the per-slot sums by T'_k / SiLU' and adds them up.
#include "kans_common.h"
#include "kans_api_internal.h"
#include <algorithm>

namespace kans {
namespace {

constexpr int kBwdThreads = 256;
constexpr int kBwdO = 64;    // output rows (dW) / batch rows (dX) per workgroup
constexpr int kBwdF = 16;    // features per workgroup
constexpr int kBwdC = 16;    // contraction chunk (batch rows for dW, outputs for dX)

__device__ __forceinline__ float silu_deriv_f32(float x) {
  const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
  return s * (1.0f + x * (1.0f - s));
}

// Slot values of one input: v[0] = SiLU(x) when has_base, then T_0..T_{K-1}(clamp x),
// zero past the last slot.  Indices stay compile-time (the array lives in registers).
template <int KPM>
__device__ __forceinline__ void slot_values(float x, int K, int has_base, float* v) {
  const float t = fminf(fmaxf(x, -1.0f), 1.0f);
  const float sx = has_base ? silu_f32(x) : 0.0f;
  float a = 1.0f, b = t;  // T_{k-2}, T_{k-1} once k >= 2
#pragma unroll
  for (int s = 0; s < KPM; ++s) {
    const int k = s - has_base;
    float val;
    if (k < 0) {
      val = sx;
    } else if (k == 0) {
      val = 1.0f;
    } else if (k == 1) {
      val = t;
    } else {
      val = __builtin_fmaf(2.0f * t, b, -a);
      a = b;
      b = val;
    }
    v[s] = k < K ? val : 0.0f;
  }
}

template <int KPM>
__global__ void __launch_bounds__(kBwdThreads)
k_cheby_bwd_dw(const float* __restrict__ dY, const float* __restrict__ X, float* __restrict__ dW,
               float* __restrict__ dWb, float* __restrict__ db, int B, int D_in, int D_out, int K,
               int has_base) {
  __shared__ float dys[kBwdC][kBwdO];
  __shared__ __attribute__((aligned(16))) float phis[kBwdC][kBwdF][KPM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int o0 = blockIdx.x * kBwdO, i0 = blockIdx.y * kBwdF;
  const int KP = K + has_base;
  const int o = o0 + lane;
  const bool do_bias = db != nullptr && blockIdx.y == 0 && wave == 0;

  float acc[4][KPM];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int s = 0; s < KPM; ++s) acc[f][s] = 0.0f;
  float bsum = 0.0f;

  for (int b0 = 0; b0 < B; b0 += kBwdC) {
    // dY rows b0.. (columns o0..o0+63), zero past B / D_out
#pragma unroll
    for (int r = 0; r < kBwdC / 4; ++r) {
      const int bb = wave * (kBwdC / 4) + r, b = b0 + bb;
      dys[bb][lane] = (b < B && o < D_out) ? dY[(long)b * D_out + o] : 0.0f;
    }
    // slots of the 16 x 16 (row, feature) pairs, one pair per thread
    {
      const int bb = tid / kBwdF, ff = tid % kBwdF, b = b0 + bb, i = i0 + ff;
      float v[KPM];
#pragma unroll
      for (int s = 0; s < KPM; ++s) v[s] = 0.0f;
      if (b < B && i < D_in) slot_values<KPM>(X[(long)b * D_in + i], K, has_base, v);
#pragma unroll
      for (int s = 0; s < KPM; ++s) phis[bb][ff][s] = v[s];
    }
    __syncthreads();
    for (int bb = 0; bb < kBwdC; ++bb) {
      const float dy = dys[bb][lane];
      bsum += dy;
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const float4* p = reinterpret_cast<const float4*>(&phis[bb][wave * 4 + f][0]);
#pragma unroll
        for (int q = 0; q < KPM / 4; ++q) {
          const float4 u = p[q];
          acc[f][4 * q + 0] = __builtin_fmaf(dy, u.x, acc[f][4 * q + 0]);
          acc[f][4 * q + 1] = __builtin_fmaf(dy, u.y, acc[f][4 * q + 1]);
          acc[f][4 * q + 2] = __builtin_fmaf(dy, u.z, acc[f][4 * q + 2]);
          acc[f][4 * q + 3] = __builtin_fmaf(dy, u.w, acc[f][4 * q + 3]);
        }
      }
    }
    __syncthreads();
  }

  if (o >= D_out) return;
  if (do_bias) db[o] = bsum;
  const long Kd = (long)D_in * K;
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int i = i0 + wave * 4 + f;
    if (i >= D_in) continue;
    if (has_base) dWb[(long)o * D_in + i] = acc[f][0];
#pragma unroll
    for (int s = 0; s < KPM; ++s) {
      const int k = s - has_base;
      if (k >= 0 && k < K) dW[(long)o * Kd + (long)i * K + k] = acc[f][s];
    }
  }
  (void)KP;
}

template <int KPM>
__global__ void __launch_bounds__(kBwdThreads)
k_cheby_bwd_dx(const float* __restrict__ dY, const float* __restrict__ X, const float* __restrict__ W,
               const float* __restrict__ Wb, float* __restrict__ dX, int B, int D_in, int D_out, int K,
               int has_base) {
  __shared__ float dys[kBwdC][kBwdO];
  __shared__ __attribute__((aligned(16))) float ws[kBwdC][kBwdF][KPM];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b0 = blockIdx.x * kBwdO, i0 = blockIdx.y * kBwdF;
  const int b = b0 + lane;
  const int KP = K + has_base;
  const long Kd = (long)D_in * K;

  float acc[4][KPM];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int s = 0; s < KPM; ++s) acc[f][s] = 0.0f;

  for (int oc = 0; oc < D_out; oc += kBwdC) {
    // dY[b0.., oc..oc+15] transposed into dys[o][b]
#pragma unroll
    for (int r = 0; r < (kBwdC * kBwdO) / kBwdThreads; ++r) {
      const int e = r * kBwdThreads + tid, bb = e / kBwdC, oo = e % kBwdC;
      const int bq = b0 + bb, o = oc + oo;
      dys[oo][bb] = (bq < B && o < D_out) ? dY[(long)bq * D_out + o] : 0.0f;
    }
    // slot weights of outputs oc.. for features i0..i0+15: ws[o][f][s]
    for (int e = tid; e < kBwdC * kBwdF * KPM; e += kBwdThreads) {
      const int oo = e / (kBwdF * KPM), rem = e % (kBwdF * KPM), ff = rem / KPM, s = rem % KPM;
      const int o = oc + oo, i = i0 + ff, k = s - has_base;
      float w = 0.0f;
      if (o < D_out && i < D_in && s < KP) w = k < 0 ? Wb[(long)o * D_in + i] : W[(long)o * Kd + (long)i * K + k];
      ws[oo][ff][s] = w;
    }
    __syncthreads();
    for (int oo = 0; oo < kBwdC; ++oo) {
      const float dy = dys[oo][lane];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const float4* p = reinterpret_cast<const float4*>(&ws[oo][wave * 4 + f][0]);
#pragma unroll
        for (int q = 0; q < KPM / 4; ++q) {
          const float4 u = p[q];
          acc[f][4 * q + 0] = __builtin_fmaf(dy, u.x, acc[f][4 * q + 0]);
          acc[f][4 * q + 1] = __builtin_fmaf(dy, u.y, acc[f][4 * q + 1]);
          acc[f][4 * q + 2] = __builtin_fmaf(dy, u.z, acc[f][4 * q + 2]);
          acc[f][4 * q + 3] = __builtin_fmaf(dy, u.w, acc[f][4 * q + 3]);
        }
      }
    }
    __syncthreads();
  }

  if (b >= B) return;
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int i = i0 + wave * 4 + f;
    if (i >= D_in) continue;
    const float x = X[(long)b * D_in + i];
    float dx = has_base ? acc[f][0] * silu_deriv_f32(x) : 0.0f;
    if (x >= -1.0f && x <= 1.0f) {
      // T'_0 = 0, T'_1 = 1, T'_k = 2 T_{k-1} + 2x T'_{k-1} - T'_{k-2}
      float Tm2 = 1.0f, Tm1 = x, dm2 = 0.0f, dm1 = 1.0f;
#pragma unroll
      for (int s = 0; s < KPM; ++s) {
        const int k = s - has_base;
        if (k == 1 && k < K) dx += acc[f][s];
        if (k >= 2 && k < K) {
          const float T = __builtin_fmaf(2.0f * x, Tm1, -Tm2);
          const float d = __builtin_fmaf(2.0f * x, dm1, __builtin_fmaf(2.0f, Tm1, -dm2));
          dx = __builtin_fmaf(acc[f][s], d, dx);
          Tm2 = Tm1;
          Tm1 = T;
          dm2 = dm1;
          dm1 = d;
        }
      }
    }
    dX[(long)b * D_in + i] = dx;
  }
}

template <int KPM>
hipError_t launch_bwd(const float* dY, const float* X, const float* W, const float* Wb, float* dW, float* dWb,
                      float* db, float* dX, int B, int D_in, int D_out, int K, int has_base, hipStream_t st) {
  const dim3 gw((D_out + kBwdO - 1) / kBwdO, (D_in + kBwdF - 1) / kBwdF);
  hipLaunchKernelGGL((k_cheby_bwd_dw<KPM>), gw, dim3(kBwdThreads), 0, st, dY, X, dW, dWb, db, B, D_in, D_out, K,
                     has_base);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 gx((B + kBwdO - 1) / kBwdO, (D_in + kBwdF - 1) / kBwdF);
  hipLaunchKernelGGL((k_cheby_bwd_dx<KPM>), gx, dim3(kBwdThreads), 0, st, dY, X, W, Wb, dX, B, D_in, D_out, K,
                     has_base);
  return hipGetLastError();
}

}  // namespace

// Slots per feature padded to the instantiated register tile.
hipError_t launch_cheby_backward(const float* dY, const float* X, const float* W, const float* Wb, float* dW,
                                 float* dWb, float* db, float* dX, int B, int D_in, int D_out, int K, int has_base,
                                 hipStream_t st) {
  const int KP = K + has_base;
  if (KP <= 4) return launch_bwd<4>(dY, X, W, Wb, dW, dWb, db, dX, B, D_in, D_out, K, has_base, st);
  if (KP <= 8) return launch_bwd<8>(dY, X, W, Wb, dW, dWb, db, dX, B, D_in, D_out, K, has_base, st);
  if (KP <= 12) return launch_bwd<12>(dY, X, W, Wb, dW, dWb, db, dX, B, D_in, D_out, K, has_base, st);
  if (KP <= 16) return launch_bwd<16>(dY, X, W, Wb, dW, dWb, db, dX, B, D_in, D_out, K, has_base, st);
  if (KP <= 24) return launch_bwd<24>(dY, X, W, Wb, dW, dWb, db, dX, B, D_in, D_out, K, has_base, st);
  return launch_bwd<36>(dY, X, W, Wb, dW, dWb, db, dX, B, D_in, D_out, K, has_base, st);
}

}  // namespace kans

using namespace kans;

namespace {

int check_bwd(const void* dY, const void* X, const void* W, const void* Wb, const void* dW, const void* dWb,
              const void* dX, int B, int D_in, int D_out, int K, int has_base, int has_bias) {
  if (!dY || !X || !W || !dW || !dX) return kans_fail(KANS_ERR_ARG, "null dY, X, W, dW or dX");
  if (B <= 0 || D_in <= 0 || D_out <= 0 || K <= 0 || K > kMaxK)
    return kans_fail(KANS_ERR_ARG, "bad dims B=%d D_in=%d D_out=%d K=%d (1 <= K <= %d)", B, D_in, D_out, K, kMaxK);
  if ((has_base != 0 && has_base != 1) || (has_bias != 0 && has_bias != 1))
    return kans_fail(KANS_ERR_ARG, "has_base / has_bias must be 0 or 1");
  if (has_base && (!Wb || !dWb)) return kans_fail(KANS_ERR_ARG, "has_base=1 but W_base or dW_base is null");
  return 0;
}

// Host-pointer backward: stage through device buffers, run, copy the gradients back.
int backward_host(const float* dY, const float* X, const float* W, const float* Wb, float* dW, float* dWb,
                  float* db, float* dX, int B, int D_in, int D_out, int K, int has_base, int has_bias) {
  int rc = check_bwd(dY, X, W, Wb, dW, dWb, dX, B, D_in, D_out, K, has_base, has_bias);
  if (rc) return rc;
  if (has_bias && !db) return kans_fail(KANS_ERR_ARG, "has_bias=1 but dbias is null");
  std::lock_guard<std::mutex> lk(kans_mutex());
  if ((rc = kans_ensure_init())) return rc;
  static DevBuf buf;
  const size_t nY = (size_t)B * D_out, nX = (size_t)B * D_in, nW = (size_t)D_out * D_in * K,
               nWb = has_base ? (size_t)D_out * D_in : 0, nb = has_bias ? (size_t)D_out : 0;
  const size_t total = nY + 2 * nX + 2 * nW + 2 * nWb + nb;
  if ((rc = buf.reserve(total * sizeof(float)))) return rc;
  float* p = (float*)buf.p;
  float *d_dY = p, *d_X = d_dY + nY, *d_W = d_X + nX, *d_Wb = d_W + nW, *d_dW = d_Wb + nWb,
        *d_dWb = d_dW + nW, *d_db = d_dWb + nWb, *d_dX = d_db + nb;
  hipStream_t st = kans_default_stream();
  HIP_TRY(hipMemcpyAsync(d_dY, dY, nY * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(d_X, X, nX * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(d_W, W, nW * 4, hipMemcpyHostToDevice, st));
  if (has_base) HIP_TRY(hipMemcpyAsync(d_Wb, Wb, nWb * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(launch_cheby_backward(d_dY, d_X, d_W, has_base ? d_Wb : nullptr, d_dW, has_base ? d_dWb : nullptr,
                                has_bias ? d_db : nullptr, d_dX, B, D_in, D_out, K, has_base, st));
  HIP_TRY(hipMemcpyAsync(dW, d_dW, nW * 4, hipMemcpyDeviceToHost, st));
  if (has_base) HIP_TRY(hipMemcpyAsync(dWb, d_dWb, nWb * 4, hipMemcpyDeviceToHost, st));
  if (has_bias) HIP_TRY(hipMemcpyAsync(db, d_db, nb * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipMemcpyAsync(dX, d_dX, nX * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return 0;
}

}  // namespace

extern "C" {

int kans_cheby_backward(const float* dY, const float* X, const float* W, const float* W_base, float* dW,
                        float* dW_base, float* dbias, float* dX, int B, int D_in, int D_out, int K, int has_base,
                        int has_bias, void* stream) {
  int rc = check_bwd(dY, X, W, W_base, dW, dW_base, dX, B, D_in, D_out, K, has_base, has_bias);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(kans_mutex());
  if ((rc = kans_ensure_init())) return rc;
  hipStream_t st = stream ? (hipStream_t)stream : kans_default_stream();
  HIP_TRY(launch_cheby_backward(dY, X, W, has_base ? W_base : nullptr, dW, has_base ? dW_base : nullptr,
                                has_bias ? dbias : nullptr, dX, B, D_in, D_out, K, has_base, st));
  return 0;
}

int metal_kan_cheby_backward_fused(const float* dY, const float* X, const float* W_cheby, const float* W_base,
                                   float* dW_cheby, float* dW_base, float* dbias, float* dX, int B, int D_in,
                                   int D_out, int degree, int has_base, int has_bias) {
  return backward_host(dY, X, W_cheby, W_base, dW_cheby, dW_base, dbias, dX, B, D_in, D_out, degree, has_base,
                       has_bias);
}

int metal_kan_cheby_backward(const float* dY, const float* X, const float* W_cheby, const float* W_base,
                             float* dW_cheby, float* dW_base, float* dbias, float* dX, int B, int D_in, int D_out,
                             int degree, int has_base, int has_bias) {
  return backward_host(dY, X, W_cheby, W_base, dW_cheby, dW_base, dbias, dX, B, D_in, D_out, degree, has_base,
                       has_bias);
}

}  // extern "C"
