// Quantized decode kernels (kans_qgemv.hip): launch descriptors shared with
// the runtime.
#pragma once
#include <hip/hip_runtime.h>
#include "kans_common.h"

namespace kans {

enum QuantKind { Q_INT4 = 0, Q_TERN = 1, Q_INT8 = 2 };

// Reduction indices per superchunk (one wave load of a 16-row block).
constexpr int kQSuper = 128;

// Batches up to kSmallB take the small-batch GEMV k_qgemv (batch rows
// replicated across the MFMA rows, three- or four-deep register ring); larger ones up to
// 32 the workgroup GEMV k_qgemv_wg (activations shared through LDS).
constexpr int kSmallB = 2;
// Work items (waves) per CU the split-K aims for (swept on the config-5
// block): small batches 8 for every format (resident: 12; 6, 7, 12 and 16
// were slower), the workgroup kernel 10 (4 to 18 measured within 1 %).
inline int items_per_cu(int /*quant*/, int B) { return B <= kSmallB ? 8 : 10; }

// 16-row blocks per decode wave (64 output rows: each activation fragment
// serves 4 weight tiles, and a wave reads 4 KB of INT4 codes per superchunk).
constexpr int kQNW = 4;
inline int qrow_blocks(int /*D_out*/) { return kQNW; }

// Register-ring slots of the small-batch GEMV k_qgemv (superchunks in flight
// while one is multiplied: depth - 1).  Three for every format: deeper rings
// measured slower on the config-5 blocks at B = 1 (INT4 depth 4 / 5: 83.4 /
// 82.0 us against 75.5; ternary depth 5 / 7: 61.0 / 63.5 against 52.6).
__host__ __device__ constexpr int qring_depth(int /*quant*/) { return 3; }

// Formats with a group affine (scale, bias) per 64 indices: INT4 and INT8 (the
// kernels apply it to the fp32 accumulator with the group sums S of Phi).
__host__ __device__ constexpr bool q_affine(int quant) { return quant != Q_TERN; }

// Bytes of one 16-row x 128-index code tile, and of one record: the kQNW code
// tiles a decode wave reads for one superchunk followed by their group
// parameters (kQNW x 16 rows x float4), so the wave's whole input is one
// contiguous stream.
__host__ __device__ constexpr int qtile_bytes(int quant) { return quant == Q_INT4 ? 1024 : quant == Q_INT8 ? 2048 : 512; }
__host__ __device__ constexpr int qrec_bytes(int quant) { return kQNW * (qtile_bytes(quant) + 16 * 16); }

// Activation basis of one layer input (see k_prep).
struct QPrep {
  const void* X;   // [B][ldx], fp32 / fp16 / bf16
  int x_dtype;
  long ldx;
  int B, MP;       // batch rows (written), allocated rows MP = 16 or 32
  int D_in, K, has_base;
  int Cb, C_tot;   // superchunks of the basis segment and of basis + base
  _Float16* Phi;   // [MP][C_tot * 128]
  float2* S;       // [C_tot][MP] (INT4 / INT8; may be null for ternary)
  int basis = BASIS_CHEBY;  // BASIS_CHEBY / BASIS_RBF / BASIS_BSPLINE
  BasisParams bp{};         // RBF centres and neg_l, B-spline grid (bp.K = K)
};

// What a small-batch decode GEMV does after its split-K partial sums are
// written (k_qgemv).  QEPI_PART stops there (separate kernels reduce them);
// QEPI_SWIGLU (GatedKAN gate | up, matrices 0 / 1 with h rows each): the last
// wave to finish output group j = gate row group j + up row group j (features
// 64j .. 64j+63; arrivals counted in `counters`) reduces the group's partials
// itself into hidden = SiLU(gate + bias) * (up + bias_u), as k_qswiglu, and
// writes the down layer's activation basis Phi2 / S2 for those features, as
// k_prep would compute it from hidden.  This replaces two kernel launches; the
// last wave pays two memory round trips (its own stores, the arrival count)
// before it reads 2 * ksplit partials per feature in batches of 8.
enum QEpiKind { QEPI_PART = 0, QEPI_SWIGLU = 2 };
constexpr int kMaxEpiSplit = 64;
// Arrival counters sit kCntStride ints (128 bytes) apart.  Every wave of a
// launch arrives at about the same time, and counters packed into a few cache
// lines serialise those atomics at ~6 ns each.  Measured: the spacing saves
// ~1 us on the ternary GatedKAN block at B = 1; a trial split-K reduce
// epilogue with 64 arrivals per group lost 25 us without it.  Wider spacing
// (1 KB, 4 KB) gained nothing more.
constexpr int kCntStride = 32;

struct QEpi {
  int kind = QEPI_PART;
  int* counters = nullptr;   // output group j at counters[j * kCntStride], 0 between launches
  const void* bias = nullptr;  // gate bias
  int bias_dtype = 0;
  const void* bias_u = nullptr;  // up bias
  int bias_u_dtype = 0;
  int round16 = 0;           // rounding of gate / up / hidden, as k_qswiglu
  int K2 = 0, has_base2 = 0, Cb2 = 0, C_tot2 = 0;  // down layer's basis geometry
  _Float16* Phi2 = nullptr;  // down layer's Phi / S (layout of QPrep)
  float2* S2 = nullptr;
};

// One decode GEMV launch over one matrix or two matrices sharing the
// activations (GatedKAN gate | up), see k_qgemv.
struct QGemv {
  const void* rec0; int D_out0;
  const void* rec1; int D_out1;  // rec1 null: single matrix
  int nw;          // 16-row blocks per row group (qrow_blocks)
  int rg_split;    // row groups of matrix 0
  int n_rg;        // row groups in total
  int ksplit;      // superchunk ranges per row group
  int C_tot;
  const _Float16* Phi;
  const float2* S;
  int B, MP;
  float* part;     // [ksplit][B][N_total] partial sums (matrix 1's columns after matrix 0's)
  int N_total;
  int nt = 0;      // non-temporal weight-record loads (see load_rec)
  QEpi epi;        // k_qgemv (B <= kSmallB) only
  // In-kernel activation basis (k_qgemv only, qgemv_pre_fits): with X set,
  // every wave computes Phi / S of its own superchunk range from the layer
  // input X into LDS, as k_prep would, and Phi / S are not read.
  const void* X = nullptr;
  int x_dtype = 0;
  long ldx = 0;
  int D_in = 0, K = 0, has_base = 0, Cb = 0;
};

// Whether the in-kernel basis fits LDS for this launch shape.
bool qgemv_pre_fits(int qt, int B, int C_tot, int ksplit, int epi_kind);

// Re-tile a packed matrix (C superchunks starting at superchunk c_off) into the records R.
hipError_t qtile_int4(const unsigned char* qw, const float* scales, const float* biases, int D_out, long rowbytes,
                      int gpr, int nrb, int C, int c_off, int C_tot, void* R, hipStream_t st);
hipError_t qtile_int8(const unsigned char* qw, const float* scales, const float* biases, int D_out, long rowbytes,
                      int gpr, int nrb, int C, int c_off, int C_tot, void* R, hipStream_t st);
hipError_t qtile_tern(const unsigned* wp, const float* scales, int D_out, int wpr, long K_dim, int gpr, int nrb,
                      int C, int c_off, int C_tot, void* R, hipStream_t st);
hipError_t qprep(int qt, const QPrep& P, hipStream_t st);
hipError_t qgemv(int qt, const QGemv& G, hipStream_t st);
// SwiGLU of gate|up split-K partials ([ksplit][B][2h]) into the down layer's
// Phi / S (E.Phi2, E.S2, geometry in E), as the fused epilogue does.
hipError_t qswiglu_basis(int qt, const QEpi& E, const float* part, int ksplit, int B, int MP, int h,
                         hipStream_t st);
// out[m][n] = sum_ks part[ks][m][n] + bias[n]
hipError_t qreduce(const float* part, int ksplit, int B, int N, const void* bias, int bias_dtype, void* Y, int y_dtype,
                   long ldy, hipStream_t st);
// hidden[m][i] = SiLU(gate) * up from the [gate | up] partials (+ biases), see k_qswiglu
hipError_t qswiglu(const float* part, int ksplit, int B, int h, const void* bias_g, int bias_g_dtype,
                   const void* bias_u, int bias_u_dtype, int round16, float* hidden, hipStream_t st);

}  // namespace kans
