// Weight quantizers (host, multi-threaded) and bit-exact dequantizers (gfx950).
//
// Formats (reference: metal_kans/quantization.py):
//   INT8 / INT4 block-affine, groups of `group_size` consecutive weights of the
//   zero-padded row-major matrix (quantization.py:24-35):
//     scale = max(max - min, 1e-7) / (2^bits - 1), bias = min            (:77-83)
//     q = clip(round_half_even((w - bias) / scale), 0, 2^bits - 1)       (:85-86)
//     INT4: two codes per byte, even index in the low nibble             (:94-97)
//     dequant = fl(fl(q * scale) + bias)  (two fp32 roundings, :146)
//   Ternary, per (row, group) over each row of K_dim weights, no padding
//   (:196-246): scale = fp32 mean(|w|) with NumPy's pairwise summation
//   (1e-4 if the mean is 0); code 0 if w/scale < -0.5, 2 if > 0.5, else 1;
//   16 codes per uint32, code k at bits 2*(k%16); dequant {-1,0,+1,0}[code]*scale
//   (:275-286, fused_kan.metal:2392-2416).
//
// The quantizers follow the reference's NumPy fallback (the path it takes on
// Linux), not its C++ bridge, which rounds half-up via a reciprocal
// (metal_kan_bridge.mm:4201-4207).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "kans_api_internal.h"

using namespace kans;

namespace {

// Run f(begin, end) over [0, n) on up to 16 host threads.
template <typename F>
void parallel_for(long n, long grain, F f) {
  unsigned hw = std::thread::hardware_concurrency();
  long nt = std::min<long>(hw ? hw : 1, 16);
  nt = std::min<long>(nt, (n + grain - 1) / grain);
  if (nt <= 1) {
    f(0L, n);
    return;
  }
  std::vector<std::thread> th;
  long chunk = (n + nt - 1) / nt;
  for (long i = 0; i < nt; ++i) {
    long b = i * chunk, e = std::min(n, b + chunk);
    if (b < e) th.emplace_back([=] { f(b, e); });
  }
  for (auto& t : th) t.join();
}

#pragma clang fp contract(off)
// NumPy's float32 pairwise summation (what np.add.reduce / np.mean use on a
// contiguous float32 run): blocks of <= 128 use eight interleaved partial sums.
float np_pairwise_sum(const float* a, long n) {
  if (n < 8) {
    float res = 0.0f;
    for (long i = 0; i < n; ++i) res += a[i];
    return res;
  }
  if (n <= 128) {
    float r[8];
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    long i = 8;
    for (; i < n - (n % 8); i += 8)
      for (int j = 0; j < 8; ++j) r[j] += a[i + j];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; ++i) res += a[i];
    return res;
  }
  long n2 = n / 2;
  n2 -= n2 % 8;
  return np_pairwise_sum(a, n2) + np_pairwise_sum(a + n2, n - n2);
}

void quantize_affine(const float* w, uint8_t* q, float* scales, float* biases, long ngroups, int gs, int bits) {
  const int max_int = (1 << bits) - 1;
  const float fmax_int = (float)max_int;
  parallel_for(ngroups, 4096, [&](long g0, long g1) {
    std::vector<int> codes(gs);
    for (long g = g0; g < g1; ++g) {
      const float* grp = w + g * gs;
      float mn = grp[0], mx = grp[0];
      for (int i = 1; i < gs; ++i) {
        mn = std::min(mn, grp[i]);
        mx = std::max(mx, grp[i]);
      }
      float range = std::max(mx - mn, 1e-7f);
      float scale = range / fmax_int;
      scales[g] = scale;
      biases[g] = mn;
      for (int i = 0; i < gs; ++i) {
        float r = std::nearbyint((grp[i] - mn) / scale);  // round half to even
        int c = (int)r;
        codes[i] = c < 0 ? 0 : (c > max_int ? max_int : c);
      }
      if (bits == 8) {
        for (int i = 0; i < gs; ++i) q[g * gs + i] = (uint8_t)codes[i];
      } else {
        uint8_t* qg = q + g * (gs / 2);
        for (int i = 0; i < gs / 2; ++i) qg[i] = (uint8_t)(codes[2 * i] | (codes[2 * i + 1] << 4));
      }
    }
  });
}

void quantize_ternary(const float* W, uint32_t* packed, float* scales, int D_out, int K_dim, int gs) {
  const int words = (K_dim + 15) / 16;
  const int gpr = (K_dim + gs - 1) / gs;
  parallel_for(D_out, 64, [&](long j0, long j1) {
    std::vector<float> absw(gs);
    for (long j = j0; j < j1; ++j) {
      const float* row = W + j * (long)K_dim;
      uint32_t* prow = packed + j * (long)words;
      std::memset(prow, 0, sizeof(uint32_t) * words);
      for (int g = 0; g < gpr; ++g) {
        const int start = g * gs, end = std::min(start + gs, K_dim), n = end - start;
        for (int i = 0; i < n; ++i) absw[i] = std::fabs(row[start + i]);
        float mean = np_pairwise_sum(absw.data(), n) / (float)n;
        float sc = mean > 0.0f ? mean : 1e-4f;
        scales[j * (long)gpr + g] = sc;
        for (int k = start; k < end; ++k) {
          float nv = row[k] / sc;
          uint32_t code = nv < -0.5f ? 0u : (nv > 0.5f ? 2u : 1u);
          prow[k / 16] |= code << ((k % 16) * 2);
        }
      }
    }
  });
}
#pragma clang fp contract(on)

// ---------------------------------------------------------------------------
// Device dequantizers: exact fp32 results of the reference dequantizers.  The
// multiply and the add are separate roundings (no FMA contraction), as NumPy's
// q * scale + bias performs them.
// ---------------------------------------------------------------------------
#pragma clang fp contract(off)
__global__ void k_dequant_int8(const uint8_t* __restrict__ q, const float* __restrict__ s,
                               const float* __restrict__ b, float* __restrict__ out, long n, int gs) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long g = i / gs;
    const float prod = (float)q[i] * s[g];
    out[i] = prod + b[g];
  }
}

__global__ void k_dequant_int4(const uint8_t* __restrict__ q, const float* __restrict__ s,
                               const float* __restrict__ b, float* __restrict__ out, long n, int gs) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long g = i / gs;
    const uint8_t byte = q[i >> 1];
    const unsigned code = (i & 1) ? (byte >> 4) : (byte & 0x0F);
    const float prod = (float)code * s[g];
    out[i] = prod + b[g];
  }
}

__global__ void k_dequant_ternary(const uint32_t* __restrict__ packed, const float* __restrict__ s,
                                  float* __restrict__ out, int D_out, int K_dim, int gs) {
  const int words = (K_dim + 15) / 16;
  const int gpr = (K_dim + gs - 1) / gs;
  const long n = (long)D_out * K_dim;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long j = i / K_dim;
    const int k = (int)(i - j * K_dim);
    const unsigned code = (packed[j * words + k / 16] >> ((k % 16) * 2)) & 3u;
    const float v = code < 3 ? (float)code - 1.0f : 0.0f;
    out[i] = v * s[j * gpr + k / gs];
  }
}

#pragma clang fp contract(on)

// SwiGLU (g * sigmoid(clamp(g, +-20))) * u  (reference: fused_kan.metal:2284-2296).
__global__ void k_swiglu_f32(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ out,
                             long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const float gv = g[i];
    const float c = fminf(fmaxf(gv, -20.0f), 20.0f);
    const float sig = 1.0f / (1.0f + expf(-c));
    out[i] = (gv * sig) * u[i];
  }
}

// Plain streaming copy (16-byte vectors); used to calibrate hardware byte
// counters against a kernel of known traffic.
__global__ void k_copy_u4(const uint4* __restrict__ src, uint4* __restrict__ dst, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

inline int grid_for(long n) { return (int)std::min<long>((n + 255) / 256, 65536); }

}  // namespace

namespace kans {
int dequant_affine_device(const void* q, const float* s, const float* b, float* out, long ngroups, int gs, int bits,
                          hipStream_t st) {
  const long n = ngroups * gs;
  if (bits == 8)
    hipLaunchKernelGGL(k_dequant_int8, dim3(grid_for(n)), dim3(256), 0, st, (const uint8_t*)q, s, b, out, n, gs);
  else
    hipLaunchKernelGGL(k_dequant_int4, dim3(grid_for(n)), dim3(256), 0, st, (const uint8_t*)q, s, b, out, n, gs);
  HIP_TRY(hipGetLastError());
  return 0;
}
int dequant_ternary_device(const uint32_t* p, const float* s, float* out, int D_out, int K_dim, int gs,
                           hipStream_t st) {
  const long n = (long)D_out * K_dim;
  hipLaunchKernelGGL(k_dequant_ternary, dim3(grid_for(n)), dim3(256), 0, st, p, s, out, D_out, K_dim, gs);
  HIP_TRY(hipGetLastError());
  return 0;
}
}  // namespace kans

// Host round trip helper: upload inputs, run `launch`, download the output.
namespace {
struct Dev {
  void* p = nullptr;
  ~Dev() { if (p) (void)hipFree(p); }
};
}  // namespace

extern "C" {

int metal_kan_quantize_int8(const float* w, uint8_t* q, float* scales, float* biases, int num_groups,
                            int group_size) {
  if (!w || !q || !scales || !biases || num_groups <= 0 || group_size <= 0)
    return kans_fail(KANS_ERR_ARG, "quantize_int8: bad argument");
  quantize_affine(w, q, scales, biases, num_groups, group_size, 8);
  return 0;
}

int metal_kan_quantize_int4(const float* w, uint8_t* q, float* scales, float* biases, int num_groups,
                            int group_size) {
  if (!w || !q || !scales || !biases || num_groups <= 0 || group_size <= 0 || (group_size & 1))
    return kans_fail(KANS_ERR_ARG, "quantize_int4: bad argument (group_size must be even)");
  quantize_affine(w, q, scales, biases, num_groups, group_size, 4);
  return 0;
}

int metal_kan_quantize_ternary(const float* W, uint32_t* packed, float* scales, int D_out, int K_dim,
                               int group_size) {
  if (!W || !packed || !scales || D_out <= 0 || K_dim <= 0 || group_size <= 0)
    return kans_fail(KANS_ERR_ARG, "quantize_ternary: bad argument");
  quantize_ternary(W, packed, scales, D_out, K_dim, group_size);
  return 0;
}

static int dequant_affine_host(const uint8_t* q, const float* s, const float* b, float* out, int ngroups, int gs,
                               int bits) {
  if (!q || !s || !b || !out || ngroups <= 0 || gs <= 0 || (bits == 4 && (gs & 1)))
    return kans_fail(KANS_ERR_ARG, "dequantize_int%d: bad argument", bits);
  int rc = kans_init();
  if (rc) return rc;
  hipStream_t st = kans_default_stream();
  const size_t qbytes = (size_t)ngroups * gs / (bits == 8 ? 1 : 2);
  const size_t pbytes = (size_t)ngroups * sizeof(float);
  const size_t obytes = (size_t)ngroups * gs * sizeof(float);
  Dev dq, ds, db, dout;
  HIP_TRY(hipMalloc(&dq.p, qbytes));
  HIP_TRY(hipMalloc(&ds.p, pbytes));
  HIP_TRY(hipMalloc(&db.p, pbytes));
  HIP_TRY(hipMalloc(&dout.p, obytes));
  HIP_TRY(hipMemcpyAsync(dq.p, q, qbytes, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(ds.p, s, pbytes, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(db.p, b, pbytes, hipMemcpyHostToDevice, st));
  if ((rc = dequant_affine_device(dq.p, (const float*)ds.p, (const float*)db.p, (float*)dout.p, ngroups, gs, bits,
                                  st)))
    return rc;
  HIP_TRY(hipMemcpyAsync(out, dout.p, obytes, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return 0;
}

int metal_kan_dequantize_int8(const uint8_t* q, const float* scales, const float* biases, float* out,
                              int num_groups, int group_size) {
  return dequant_affine_host(q, scales, biases, out, num_groups, group_size, 8);
}

int metal_kan_dequantize_int4(const uint8_t* q, const float* scales, const float* biases, float* out,
                              int num_groups, int group_size) {
  return dequant_affine_host(q, scales, biases, out, num_groups, group_size, 4);
}

int metal_kan_dequantize_ternary(const uint32_t* packed, const float* scales, float* out, int D_out, int K_dim,
                                 int group_size) {
  if (!packed || !scales || !out || D_out <= 0 || K_dim <= 0 || group_size <= 0)
    return kans_fail(KANS_ERR_ARG, "dequantize_ternary: bad argument");
  int rc = kans_init();
  if (rc) return rc;
  hipStream_t st = kans_default_stream();
  const size_t pbytes = (size_t)D_out * ((K_dim + 15) / 16) * sizeof(uint32_t);
  const size_t sbytes = (size_t)D_out * ((K_dim + group_size - 1) / group_size) * sizeof(float);
  const size_t obytes = (size_t)D_out * K_dim * sizeof(float);
  Dev dp, ds, dout;
  HIP_TRY(hipMalloc(&dp.p, pbytes));
  HIP_TRY(hipMalloc(&ds.p, sbytes));
  HIP_TRY(hipMalloc(&dout.p, obytes));
  HIP_TRY(hipMemcpyAsync(dp.p, packed, pbytes, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(ds.p, scales, sbytes, hipMemcpyHostToDevice, st));
  if ((rc = dequant_ternary_device((const uint32_t*)dp.p, (const float*)ds.p, (float*)dout.p, D_out, K_dim,
                                   group_size, st)))
    return rc;
  HIP_TRY(hipMemcpyAsync(out, dout.p, obytes, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return 0;
}

// Device-pointer dequantizers (enqueued on `stream`, NULL = library stream).
int kans_dequantize_affine_device(const void* q, const float* scales, const float* biases, float* out,
                                  long num_groups, int group_size, int bits, void* stream) {
  if (!q || !scales || !biases || !out || num_groups <= 0 || group_size <= 0 || (bits != 8 && bits != 4))
    return kans_fail(KANS_ERR_ARG, "dequantize_affine_device: bad argument");
  int rc = kans_init();
  if (rc) return rc;
  return dequant_affine_device(q, scales, biases, out, num_groups, group_size, bits,
                               stream ? (hipStream_t)stream : kans_default_stream());
}

int kans_dequantize_ternary_device(const uint32_t* packed, const float* scales, float* out, int D_out, int K_dim,
                                   int group_size, void* stream) {
  if (!packed || !scales || !out || D_out <= 0 || K_dim <= 0 || group_size <= 0)
    return kans_fail(KANS_ERR_ARG, "dequantize_ternary_device: bad argument");
  int rc = kans_init();
  if (rc) return rc;
  return dequant_ternary_device(packed, scales, out, D_out, K_dim, group_size,
                                stream ? (hipStream_t)stream : kans_default_stream());
}

// Device copy of `bytes` (multiple of 16, 16-byte aligned pointers) with a plain kernel.
int kans_copy_device(void* dst, const void* src, size_t bytes, void* stream) {
  if (!dst || !src || (bytes & 15) || (((uintptr_t)dst | (uintptr_t)src) & 15))
    return kans_fail(KANS_ERR_ARG, "copy: bad argument");
  int rc = kans_init();
  if (rc) return rc;
  const long n = (long)(bytes / 16);
  hipLaunchKernelGGL(k_copy_u4, dim3(std::min<long>((n + 255) / 256, 8192)), dim3(256), 0,
                     stream ? (hipStream_t)stream : kans_default_stream(), (const uint4*)src, (uint4*)dst, n);
  HIP_TRY(hipGetLastError());
  return 0;
}

// replaces metal_kan_swiglu_forward (metal_kan_bridge.mm:4846-4875)
int metal_kan_swiglu_forward(const float* gate, const float* up, float* out, int n) {
  if (!gate || !up || !out || n <= 0) return kans_fail(KANS_ERR_ARG, "swiglu: bad argument");
  int rc = kans_init();
  if (rc) return rc;
  hipStream_t st = kans_default_stream();
  const size_t bytes = (size_t)n * sizeof(float);
  Dev dg, du, dout;
  HIP_TRY(hipMalloc(&dg.p, bytes));
  HIP_TRY(hipMalloc(&du.p, bytes));
  HIP_TRY(hipMalloc(&dout.p, bytes));
  HIP_TRY(hipMemcpyAsync(dg.p, gate, bytes, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(du.p, up, bytes, hipMemcpyHostToDevice, st));
  hipLaunchKernelGGL(k_swiglu_f32, dim3(grid_for(n)), dim3(256), 0, st, (const float*)dg.p, (const float*)du.p,
                     (float*)dout.p, (long)n);
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipMemcpyAsync(out, dout.p, bytes, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return 0;
}

}  // extern "C"
