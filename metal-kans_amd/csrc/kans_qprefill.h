// Quantized prefill kernels (kans_qprefill.hip): tile format and launch
// descriptors shared with the runtime.
#pragma once
#include <hip/hip_runtime.h>
#include "kans_common.h"

namespace kans {

// Prefill tile format of one quantized matrix segment (the basis matrix
// W [D_out][D_in*K], or the base matrix W_base [D_out][D_in] with K = 1), built
// once from the reference's packed arrays:
//   codes  C[fb][ob][s][lane]: the 8 codes of chunk (output o = 32 ob + lane % 32,
//          features 16 fb + 8 (lane / 32) + e, e = 0..7, slot s < K), padded
//          rows / features hold code 0 (ternary: code 1, a zero weight);
//          INT4: one dword, code e at bit kInt4Pos[e];
//          INT8: two dwords, code e in byte e;
//          ternary: K even -- C[fb][ob][s/2][lane] is a dword holding slots s
//          (layout A: code 2p at bit 2p, 2p+1 at bit 16+2p) and s+1 (layout B:
//          bits 8+2p, 24+2p); K = 1 -- 16 bits, code 2p at bit 2p, code 2p+1 at
//          bit 8+2p;
//   params P[g][o]: the reference's group parameters, group g = j / group_size
//          of the row's reduction index j = i*K + s; (scale, bias) float2 for
//          INT8 / INT4 (group 64), scale float for ternary (group 32).
// With K in {1, 2, 4, 8} the 8 codes of a chunk (features i0 .. i0 + 7 of one
// slot, reduction indices i K + s) lie in one group of 64 (INT8 / INT4), and
// in one group of 32 (ternary) except at K = 8, where codes 0-3 and 4-7 fall
// in consecutive groups: the fused kernel loads one parameter set per chunk,
// two for ternary at K = 8.  Other K (a chunk straddling a group boundary at a
// data-dependent position) are not built.  Bases: Chebyshev for every such K;
// the Gaussian RBF on uniform centres (the recurrence of BasisGen<BASIS_RBF_REC>)
// and the cubic B-spline for K in {4, 8} (FastKAN's and BSplineKAN's default
// K = 8), except INT8 B-spline at K = 8: with the code words of a whole block
// in registers that kernel spills (measured 2.2x the dense fp16 kernel's time
// on the dequantized weights, where the other K = 8 kernels take 1.09-1.21x,
// INT8 Chebyshev 1.38x).
__host__ __device__ constexpr int qp_chunk_bytes(int qt) { return qt == 0 ? 4 : qt == 2 ? 8 : 2; }  // Q_INT4/TERN/INT8
__host__ __device__ constexpr int qp_group(int qt) { return qt == 1 ? 32 : 64; }
__host__ __device__ constexpr int qp_param_floats(int qt) { return qt == 1 ? 1 : 2; }
inline bool qp_supported(int qt, int K, int basis = BASIS_CHEBY, int rbf_rec = 1) {
  if (basis == BASIS_CHEBY) return K == 1 || K == 2 || K == 4 || K == 8;
  if (basis == BASIS_RBF && !rbf_rec) return false;
  if (basis == BASIS_BSPLINE && K == 8 && qt == 2 /* Q_INT8 */) return false;
  return K == 4 || K == 8;
}

enum QPEpi { QP_EPI_PLAIN = 0, QP_EPI_SWIGLU = 1 };

// One quantized matrix as the fused kernel reads it.
struct QPMat {
  const unsigned char* cb;  // basis codes
  const unsigned char* cw;  // base codes (has_base)
  const float* pb;          // basis parameters [G_b][ldp]
  const float* pw;          // base parameters [G_w][ldp]
  long ldp;                 // parameter row stride (nob_pad * 32 outputs)
  int nob_pad;              // 32-column blocks, padded to a multiple of 8
  int D_out;
  const void* bias;         // [D_out] (bias_dt) or null
};

// One fused prefill launch: y = forward(x) of matrix m[0] (grp = 8: all eight
// column blocks of an N-tile from m[0]), or hidden = SiLU(gate) * up of the
// column-paired gate m[0] / up m[1] (grp = 4: column blocks 0..3 of an N-tile
// from m[0], 4..7 the same columns of m[1]).
struct QPLaunch {
  int qt, K, has_base;
  int basis = BASIS_CHEBY;  // BASIS_CHEBY / BASIS_RBF (uniform centres) / BASIS_BSPLINE
  BasisParams bp{};         // RBF / B-spline parameters (bp.K = K)
  const void* X; long ldx; int x_dtype;
  QPMat m[2];
  int grp;
  int bias_dtype;
  void* Y; long ldy; int y_dtype;
  float* part;      // split workspace (splits * B * n_tiles * 256 floats) when splits > 1
  int B, D_in, splits;
  int epi, round16;
};

// Split-K workspace floats a launch needs (0 when unsplit).
long qp_part_floats(const QPLaunch& L);
// Feature splits the launcher picks for B rows (so the grid fills the GPU).
int qp_choose_splits(int B, int D_in, int n_cols, int grp);
hipError_t qp_launch(const QPLaunch& L, hipStream_t st);

// Re-tiling of the reference formats into the prefill layout (device arrays).
// affine: qw [D_out][rowbytes] (INT4 nibbles, even index low / INT8 bytes),
// scales / biases [D_out][gpr]; ternary: wp [D_out][wpr] uint32, scales [D_out][gpr].
hipError_t qp_tile_affine(int bits, const unsigned char* qw, long rowbytes, const float* scales, const float* biases,
                          int gpr, int D_out, int D_in, int Kseg, int nfb, int nob_pad, int G_alloc, void* codes,
                          float* params, hipStream_t st);
hipError_t qp_tile_tern(const unsigned* wp, int wpr, const float* scales, int gpr, int D_out, int D_in, int Kseg,
                        int nfb, int nob_pad, int G_alloc, void* codes, float* params, hipStream_t st);

}  // namespace kans
