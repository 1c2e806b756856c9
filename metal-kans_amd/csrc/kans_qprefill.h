// Quantized prefill kernels (kans_qprefill_kernel.h, launched by
// kans_qprefill.hip): tile format and launch descriptors shared with the
// runtime.
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
//          ternary: K > 1 -- C[fb][ob][s/2][lane] is a dword holding slots s
//          (layout A: code 2p at bit 2p, 2p+1 at bit 16+2p) and s+1 (layout B:
//          bits 8+2p, 24+2p), an odd K padded with one slot of zero weights;
//          K = 1 -- 16 bits, code 2p at bit 2p, code 2p+1 at bit 8+2p;
//   params P[g][o]: the reference's group parameters, group g = j / group_size
//          of the row's reduction index j = i*K + s; (scale, bias) float2 for
//          INT8 / INT4 (group 64), scale float for ternary (group 32); a few
//          zero rows past the last group (a half-block's parameter loads may
//          reach past it).
// Groups: lane half h of feature block f decodes features 16 f + 8 h .. + 7,
// whose K slots are the 8 K consecutive reduction indices from (16 f + 8 h) K
// (a half-block).  It loads the parameters of every group those indices meet
// (qp_ngroups: 1 for K in {1, 2, 4} and INT at K = 8, up to 3), and each code
// takes the group of its own index.  Where the half-block starts within its
// group repeats in f with period qp_period (1, 2 or 4), so the kernel's block
// loop is unrolled by that period and every code's group is a compile-time
// constant per lane half: the decode costs the same instructions as with one
// group, plus a lane-half select for the few codes whose group differs
// between the two halves.  K <= 9 (K + 1 slots of fp16 B-tiles fill the LDS).
// Bases: Chebyshev at every such K; the Gaussian RBF on uniform centres (the
// recurrence of BasisGen<BASIS_RBF_REC>) at K >= 2; the cubic B-spline at
// K = 4 (G = 1, per-value selection) and K = 8 (G = 5, the basis table).  Not
// built, because the kernel spills (register pressure: 100-600 spilled
// registers against 0-25 for the kinds that are built): INT8 with the base
// branch at K = 7, INT8 B-spline at K = 8 (measured 2.2x the dense fp16
// kernel's time on the dequantized weights, where the other K = 8 kernels
// take 1.09-1.21x, INT8 Chebyshev 1.38x), and the per-value B-spline at other
// G.  Such layers take the dense kernels on the dequantized weights above 32
// rows (the decode GEMVs take every basis and K).
constexpr int kQPMaxK = 9;
// offset of half-block (f, h)'s first reduction index within its group
__host__ __device__ constexpr int qp_r0(int K, int GS, int f, int h) { return ((16 * f + 8 * h) * K) % GS; }
// group of code e of slot s, relative to the half-block's first group
__host__ __device__ constexpr int qp_dg(int K, int GS, int f, int h, int s, int e) {
  return (qp_r0(K, GS, f, h) + e * K + s) / GS;
}
// the half-block's first group minus floor(16 f K / GS) (the block's first group)
__host__ __device__ constexpr int qp_gl(int K, int GS, int f, int h) { return ((16 * f * K) % GS + 8 * h * K) / GS; }
// smallest c >= 1 with 16 c K = 0 (mod GS): r0 and gl repeat with period c in f
__host__ __device__ constexpr int qp_cycle(int K, int GS) {
  int c = 1;
  while ((16 * c * K) % GS) ++c;
  return c;
}
// groups one half-block meets, at most
__host__ __device__ constexpr int qp_ngroups(int K, int GS) {
  int n = 1;
  for (int f = 0; f < qp_cycle(K, GS); ++f)
    for (int h = 0; h < 2; ++h) {
      const int m = (qp_r0(K, GS, f, h) + 8 * K - 1) / GS + 1;
      n = m > n ? m : n;
    }
  return n;
}
// phases of f the kernel tells apart: 1 when every f decodes and addresses
// its parameters alike, else qp_cycle
__host__ __device__ constexpr int qp_period(int K, int GS) {
  const int c = qp_cycle(K, GS);
  for (int f = 1; f < c; ++f)
    for (int h = 0; h < 2; ++h) {
      if (qp_gl(K, GS, f, h) != qp_gl(K, GS, 0, h)) return c;
      for (int s = 0; s < K; ++s)
        for (int e = 0; e < 8; ++e)
          if (qp_dg(K, GS, f, h, s, e) != qp_dg(K, GS, 0, h, s, e)) return c;
    }
  return 1;
}
__host__ __device__ constexpr int qp_chunk_bytes(int qt) { return qt == 0 ? 4 : qt == 2 ? 8 : 2; }  // Q_INT4/TERN/INT8
__host__ __device__ constexpr int qp_group(int qt) { return qt == 1 ? 32 : 64; }
__host__ __device__ constexpr int qp_param_floats(int qt) { return qt == 1 ? 1 : 2; }
inline bool qp_supported(int qt, int K, int has_base, int basis = BASIS_CHEBY, int rbf_rec = 1) {
  if (K < 1 || K > kQPMaxK || (qt == 2 /* Q_INT8 */ && has_base && K == 7)) return false;
  if (basis == BASIS_CHEBY) return true;
  if (basis == BASIS_RBF) return rbf_rec && K >= 2;
  return K == 4 || (K == 8 && qt != 2);
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

// Chebyshev K = 4 prefill kernels: two feature blocks per LDS stage (1, the
// default) or one (0); kans_prefill_set_block_pairs.
extern int g_qp_block_pairs;

// Split-K workspace floats a launch needs (0 when unsplit).
long qp_part_floats(const QPLaunch& L);
// Feature splits the launcher picks for B rows (so the grid fills the GPU).
int qp_choose_splits(int B, int D_in, int n_cols, int grp);
hipError_t qp_launch(const QPLaunch& L, hipStream_t st);

// Grid of one fused launch: m_tiles x n_tiles output tiles by nsp feature
// splits of fb_per_split feature blocks each.
struct QPGrid {
  int m_tiles, n_tiles, nfb, fb_per_split, nsp;
};
// The fused kernels of each weight format without / with the base branch
// (kans_qprefill_{int4,int8,tern}_b{0,1}.hip).
hipError_t qp_run_int4_b0(const QPLaunch& L, const QPGrid& G, hipStream_t st);
hipError_t qp_run_int4_b1(const QPLaunch& L, const QPGrid& G, hipStream_t st);
hipError_t qp_run_int8_b0(const QPLaunch& L, const QPGrid& G, hipStream_t st);
hipError_t qp_run_int8_b1(const QPLaunch& L, const QPGrid& G, hipStream_t st);
hipError_t qp_run_tern_b0(const QPLaunch& L, const QPGrid& G, hipStream_t st);
hipError_t qp_run_tern_b1(const QPLaunch& L, const QPGrid& G, hipStream_t st);

// Re-tiling of the reference formats into the prefill layout (device arrays).
// affine: qw [D_out][rowbytes] (INT4 nibbles, even index low / INT8 bytes),
// scales / biases [D_out][gpr]; ternary: wp [D_out][wpr] uint32, scales [D_out][gpr].
hipError_t qp_tile_affine(int bits, const unsigned char* qw, long rowbytes, const float* scales, const float* biases,
                          int gpr, int D_out, int D_in, int Kseg, int nfb, int nob_pad, int G_alloc, void* codes,
                          float* params, hipStream_t st);
hipError_t qp_tile_tern(const unsigned* wp, int wpr, const float* scales, int gpr, int D_out, int D_in, int Kseg,
                        int nfb, int nob_pad, int G_alloc, void* codes, float* params, hipStream_t st);

}  // namespace kans
