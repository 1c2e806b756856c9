// Quantized decode kernels (kans_qgemv.hip): launch descriptors shared with
// the runtime.
#pragma once
#include <hip/hip_runtime.h>

namespace kans {

enum QuantKind { Q_INT4 = 0, Q_TERN = 1 };

// Reduction indices per superchunk (one wave load of a 16-row block).
constexpr int kQSuper = 128;

// 16-row blocks per decode wave (64 output rows: each activation fragment
// serves 4 weight tiles, and a wave reads 4 KB of weights per superchunk).
inline int qrow_blocks(int /*D_out*/) { return 4; }

// Activation basis of one layer input (see k_prep).
struct QPrep {
  const void* X;   // [B][ldx], fp32 / fp16 / bf16
  int x_dtype;
  long ldx;
  int B, MP;       // batch rows, padded to MP = 16 or 32 (rows >= B are written as 0)
  int D_in, K, has_base;
  int Cb, C_tot;   // superchunks of the basis segment and of basis + base
  _Float16* Phi;   // [MP][C_tot * 128]
  float2* S;       // [C_tot][MP] (INT4 only; may be null for ternary)
};

// One decode GEMV launch over one matrix or two matrices sharing the
// activations (GatedKAN gate | up), see k_qgemv.
struct QGemv {
  const void* q0; const float4* sb0; int D_out0;
  const void* q1; const float4* sb1; int D_out1;  // q1 null: single matrix
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
};

hipError_t qtile_int4(const unsigned char* qw, const float* scales, const float* biases, int D_out, long rowbytes,
                      int gpr, int nrb, int C, int c_off, int C_tot, int nw, void* Q, float4* SB, hipStream_t st);
hipError_t qtile_tern(const unsigned* wp, const float* scales, int D_out, int wpr, long K_dim, int gpr, int nrb,
                      int C, int c_off, int C_tot, int nw, void* Q, float4* SB, hipStream_t st);
hipError_t qprep(int qt, const QPrep& P, hipStream_t st);
hipError_t qgemv(int qt, const QGemv& G, hipStream_t st);
// out[m][n] = sum_ks part[ks][m][n] + bias[n]
hipError_t qreduce(const float* part, int ksplit, int B, int N, const void* bias, int bias_dtype, void* Y, int y_dtype,
                   long ldy, hipStream_t st);
// hidden[m][i] = SiLU(gate) * up from the [gate | up] partials (+ biases), see k_qswiglu
hipError_t qswiglu(const float* part, int ksplit, int B, int h, const void* bias_g, const void* bias_u, int bias_dtype,
                   int round16, float* hidden, hipStream_t st);

}  // namespace kans
