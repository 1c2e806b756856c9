// Shared device-side definitions for the MI355X (gfx950) fused KAN kernels.
//
// Element types, MFMA fragment types, the basis generators that run inside the
// fused kernels, and the tiled weight layout shared by the repack kernel and the
// fused forward.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kans {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

enum Basis { BASIS_CHEBY = 0, BASIS_RBF = 1, BASIS_BSPLINE = 2 };
// Kernel-only basis id: the Gaussian RBF of BASIS_RBF with its scaled centres
// read from a table in LDS (BasisGen<BASIS_RBF_TABLE>); the public API never
// sees it.
constexpr int BASIS_RBF_TABLE = 3;
// Kernel-only basis id: the Chebyshev basis of BASIS_CHEBY, advanced in place
// with each step emitting the value it just computed (BasisGen<BASIS_CHEBY_POST>).
constexpr int BASIS_CHEBY_POST = 4;
enum DType { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

constexpr float kLog2e = 1.4426950408889634f;
// Maximum number of RBF centres / basis functions per input feature.
constexpr int kMaxK = 32;

// Basis parameters passed by value to the fused kernels.
struct BasisParams {
  int K;              // basis functions per feature (excluding the SiLU base slot)
  int grid_size;      // B-spline: number of intervals G (K = G + 3)
  float grid_min;     // B-spline: left end of the grid
  float inv_h;        // B-spline: G / (max - min)
  float neg_l;        // RBF: -inv_den * log2(e)
  int have_centers;   // RBF: centres set
  float rbf_s;        // RBF: sqrt(-neg_l), so phi_k = exp2(-(s*x - s*c_k)^2)
  float centers[kMaxK];  // RBF centres c_k (host copy)
  // RBF scaled centres s * c_k, by value: the kernels read them with scalar
  // loads from the argument segment, which do not wait on the vector-memory
  // counter that the weight / input prefetch uses.
  float rbf_sc[kMaxK];
};

// ---------------------------------------------------------------------------
// Tiled weight layout W'.  The contraction runs over (feature i, slot s) pairs,
// where slot 0 is the SiLU base branch when has_base and slots has_base.. are the
// K basis functions.  The inner dimension is reordered so that one MFMA step
// consumes 16 features of ONE slot:
//
//   W'[fb][s][ob][chunk][lane][e]
//     fb    = i / 16                 (feature block)
//     s     = slot                   (0 .. KP-1)
//     ob    = o / 32                 (32-column output block; padded to kObPad)
//     lane  = (o % 32) + 32 * ((i % 16) / 8)
//     j     = i % 8,  chunk = j / EPC,  e = j % EPC  (EPC = 16 / sizeof(T))
//
// so a lane's 16-byte chunk is exactly its MFMA B-operand for that slot, and one
// (fb, s) step of an N-tile of NB output blocks is NB contiguous KB-sized tiles.
// ---------------------------------------------------------------------------
constexpr int kObPad = 8;  // output blocks padded to a multiple of 8 (max NB)

__host__ __device__ inline int round_up(int a, int b) { return (a + b - 1) / b * b; }

template <typename T> struct TypeTag;
template <> struct TypeTag<_Float16> { static constexpr int dt = DT_F16; };
template <> struct TypeTag<__bf16> { static constexpr int dt = DT_BF16; };
template <> struct TypeTag<float> { static constexpr int dt = DT_F32; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(__bf16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return (_Float16)v; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float v) { return (__bf16)v; }

// SiLU on the raw input: x / (1 + e^-x)  (reference: fused_kan.metal:13-16,132-133).
__device__ __forceinline__ float silu_f32(float x) {
  float e = __builtin_amdgcn_exp2f(-x * kLog2e);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// ---------------------------------------------------------------------------
// Basis generators.  A generator holds NV input values of one lane.  ``begin``
// is called once per 16-feature block; then ``one(k, v)`` yields basis
// function k (k = 0, 1, 2, ... in order within a block) for all NV inputs in
// fp32, and ``pair(k, v0, v1)`` functions k and k+1 (k even).
// ---------------------------------------------------------------------------
template <int BASIS, int NV> struct BasisGen;

// Chebyshev T_k(clamp(x,-1,1)) by the three-term recurrence in fp32 registers
// (reference: fused_kan.metal:205-238 fp32, :1399-1426 fp16 with fma).  Two
// registers r0, r1 hold consecutive T's; a step of parity P emits r_P and
// advances it by two degrees (r_P <- 2t r_{1-P} - r_P), so consecutive steps
// alternate registers without any register rotation.  ``begin(.., swap)``
// places T_0 in r1 instead of r0 when basis 0 is emitted at an odd step.
template <int NV> struct BasisGen<BASIS_CHEBY, NV> {
  float tw[NV], r0[NV], r1[NV];
  __device__ __forceinline__ void begin(const float* x, const BasisParams&, bool swap = false) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float t = __builtin_fminf(__builtin_fmaxf(x[v], -1.0f), 1.0f);
      tw[v] = t + t;
      r0[v] = swap ? t : 1.0f;
      r1[v] = swap ? 1.0f : t;
    }
  }
  template <int P>
  __device__ __forceinline__ void step(int, const BasisParams&, float* v0) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if constexpr (P == 0) {
        v0[v] = r0[v];
        r0[v] = __builtin_fmaf(tw[v], r1[v], -r0[v]);
      } else {
        v0[v] = r1[v];
        r1[v] = __builtin_fmaf(tw[v], r0[v], -r1[v]);
      }
    }
  }
  __device__ __forceinline__ void one(int k, const BasisParams& bp, float* v0) {
    if ((k & 1) == 0) step<0>(k, bp, v0); else step<1>(k, bp, v0);
  }
  __device__ __forceinline__ void pair(int, const BasisParams&, float* v0, float* v1) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      v0[v] = r0[v];
      v1[v] = r1[v];
      r0[v] = __builtin_fmaf(tw[v], r1[v], -r0[v]);
      r1[v] = __builtin_fmaf(tw[v], r0[v], -r1[v]);
    }
  }
};

// Chebyshev T_k(clamp(x,-1,1)) as BasisGen<BASIS_CHEBY>, but each step first
// advances its register and then emits the fresh value: step<P> does
// r_P <- 2t r_{1-P} - r_P and returns r_P, so the emitted value is the result
// of the step's own fma and no copy of the previous value has to stay alive.
// Before the first step the registers hold T_{-2} = T_2 = 2t^2 - 1 and
// T_{-1} = T_1 = t (T_{-k} = T_k), which yields T_0 = 2t*t - (2t^2 - 1) and
// T_1 = 2t*T_0 - t; both are within an fp32 rounding of 1 and t, far below
// the 16-bit rounding of the MFMA operands this generator feeds.
template <int NV> struct BasisGen<BASIS_CHEBY_POST, NV> {
  float tw[NV], r0[NV], r1[NV];
  __device__ __forceinline__ void begin(const float* x, const BasisParams&, bool swap = false) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const float t = __builtin_fminf(__builtin_fmaxf(x[v], -1.0f), 1.0f);
      tw[v] = t + t;
      const float tm2 = __builtin_fmaf(tw[v], t, -1.0f);
      r0[v] = swap ? t : tm2;
      r1[v] = swap ? tm2 : t;
    }
  }
  template <int P>
  __device__ __forceinline__ void step(int, const BasisParams&, float* v0) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      // the empty asm makes the fp32 result opaque, so the packing reads it
      // instead of recomputing the fma with a 16-bit result (v_fma_mix), which
      // would keep the previous value alive and cost a register copy per value
      if constexpr (P == 0) {
        r0[v] = __builtin_fmaf(tw[v], r1[v], -r0[v]);
        asm volatile("" : "+v"(r0[v]));
        v0[v] = r0[v];
      } else {
        r1[v] = __builtin_fmaf(tw[v], r0[v], -r1[v]);
        asm volatile("" : "+v"(r1[v]));
        v0[v] = r1[v];
      }
    }
  }
};

// Gaussian RBF exp(-(x - c_k)^2 * inv_den) = exp2(-(s*x - s*c_k)^2) with
// s = sqrt(inv_den * log2(e)) (reference: fused_kan.metal:140-166,
// fast_kan.py:40-42): one fma, one multiply and one exp2 per value; s*c_k
// comes precomputed in BasisParams::rbf_sc (a kernel argument).
template <int NV> struct BasisGen<BASIS_RBF, NV> {
  float xv[NV];
  template <int P>
  __device__ __forceinline__ void step(int k, const BasisParams& bp, float* v0) { one(k, bp, v0); }
  __device__ __forceinline__ void begin(const float* x, const BasisParams&, bool = false) {
#pragma unroll
    for (int v = 0; v < NV; ++v) xv[v] = x[v];
  }
  __device__ __forceinline__ void one(int k, const BasisParams& bp, float* v0) {
    const float sck = bp.rbf_sc[k];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const float t = __builtin_fmaf(xv[v], bp.rbf_s, -sck);
      v0[v] = __builtin_amdgcn_exp2f(-(t * t));
    }
  }
  __device__ __forceinline__ void pair(int k, const BasisParams& bp, float* v0, float* v1) {
    one(k, bp, v0);
    one(k + 1, bp, v1);
  }
};

// Gaussian RBF as BasisGen<BASIS_RBF>, with the scaled centre s*c_k read from
// `tab`, a copy of BasisParams::rbf_sc in LDS (entry K = 0 for the unused step
// after a block's last slot).  A broadcast LDS read is counted with the LDS
// reads of the weights (in order), where a scalar load from the argument
// segment would force a wait for all of them.
template <int NV> struct BasisGen<BASIS_RBF_TABLE, NV> {
  float xv[NV];
  const float* tab = nullptr;
  __device__ __forceinline__ void begin(const float* x, const BasisParams&, bool = false) {
#pragma unroll
    for (int v = 0; v < NV; ++v) xv[v] = x[v];
  }
  template <int P>
  __device__ __forceinline__ void step(int k, const BasisParams& bp, float* v0) {
    const float sck = tab[k];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const float t = __builtin_fmaf(xv[v], bp.rbf_s, -sck);
      v0[v] = __builtin_amdgcn_exp2f(-(t * t));
    }
  }
};

// Clamped uniform cubic B-spline, G+3 bases, four non-zero per input
// (reference: fused_kan.metal:240-276, bspline_kan.py:40-54):
//   pos = (x - grid_min) * inv_h, span = clamp(floor(pos), 0, G-1),
//   u = clamp(pos - span, 0, 1), values at span..span+3.
template <int NV> struct BasisGen<BASIS_BSPLINE, NV> {
  float w0[NV], w1[NV], w2[NV], w3[NV];
  int span[NV];
  template <int P>
  __device__ __forceinline__ void step(int k, const BasisParams& bp, float* v0) { one(k, bp, v0); }
  __device__ __forceinline__ void begin(const float* x, const BasisParams& p, bool = false) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float pos = (x[v] - p.grid_min) * p.inv_h;
      float fl = __builtin_floorf(pos);
      fl = __builtin_fminf(__builtin_fmaxf(fl, 0.0f), (float)(p.grid_size - 1));
      float u = __builtin_fminf(__builtin_fmaxf(pos - fl, 0.0f), 1.0f);
      float om = 1.0f - u;
      float u2 = u * u, u3 = u2 * u;
      const float inv6 = 1.0f / 6.0f;
      w0[v] = om * om * om * inv6;
      w1[v] = (3.0f * u3 - 6.0f * u2 + 4.0f) * inv6;
      w2[v] = (-3.0f * u3 + 3.0f * u2 + 3.0f * u + 1.0f) * inv6;
      w3[v] = u3 * inv6;
      span[v] = (int)fl;
    }
  }
  __device__ __forceinline__ void one(int k, const BasisParams&, float* v0) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int d = k - span[v];
      float r = 0.0f;
      r = (d == 0) ? w0[v] : r;
      r = (d == 1) ? w1[v] : r;
      r = (d == 2) ? w2[v] : r;
      r = (d == 3) ? w3[v] : r;
      v0[v] = r;
    }
  }
  __device__ __forceinline__ void pair(int k, const BasisParams& bp, float* v0, float* v1) {
    one(k, bp, v0);
    one(k + 1, bp, v1);
  }
};

}  // namespace kans
