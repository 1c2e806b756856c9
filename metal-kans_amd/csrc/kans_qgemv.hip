// Fused decode (small-batch) forward of Chebyshev KAN layers whose weights are
// kept in the reference's packed INT4, INT8 or ternary formats, and of the
// GatedKAN block built from three such layers.
//
//   y[b,o] = bias[o] + sum_i SiLU(v[b,i]) Wb[o,i] + sum_{i,k} T_k(clamp v[b,i]) W[o,i*K+k]
//   W  = q*s + b per group of 64 (INT4 / INT8, quantization.py:13-99), or
//        t*s, t in {-1,0,+1} per group of 32 (ternary, quantization.py:191-246)
//
// Replaces metal_kan_forward_ternary_cheby (metal_kan_bridge.mm:4684-4733,
// fused_kan.metal:2167-2223), which has no base branch and no INT4 variant, and
// the reference GatedKAN forward on dequantized weights (gated_kan.py:86-138).
//
// At B <= 32 the layer is HBM-bound: the job is to stream the packed weights
// once at full bandwidth.  Design:
//   * the packed weights are re-tiled once on upload into MFMA B-fragment order:
//     one "superchunk" = 16 output rows x 128 reduction indices, one 16-byte
//     (INT4), two 16-byte (INT8) or one 8-byte (ternary) load per lane,
//     1 KB / 2 KB / 512 B per wave, fully coalesced; the per-group affine
//     parameters are re-tiled alongside;
//   * INT4 nibbles become fp16 with the 0x6400|q trick (the fp16 value 1024+q,
//     exact), two per v_and_or_b32; INT8 bytes become 1024+q with one
//     v_perm_b32 per pair (high byte 0x64); ternary codes become +-1/0 fp16
//     through a v_perm_b32 byte table.  The group scale is applied to the fp32
//     MFMA accumulator once per group: y += s * sum(phi*(1024+q)) + (b - 1024 s)
//     * sum(phi) for INT4 / INT8, y += s * sum(phi*t) for ternary;
//   * the activation basis phi (T_k and SiLU of the layer input, fp16, permuted
//     to match the unpack order) and its per-group sums are computed once per
//     layer into a small buffer that stays in L2; the waves read their A
//     fragments (v_mfma_f32_16x16x32_f16, 16 batch rows per tile) from there;
//   * one wave owns 4 row blocks (64 output rows) and a contiguous range of
//     superchunks (split-K over waves for memory-level parallelism); partial
//     sums go to an fp32 workspace that a small kernel reduces (+ bias), in
//     the GatedKAN block together with SwiGLU(gate, up) -- at B <= 2 the
//     gate|up GEMV's last wave per feature group does that itself;
//   * B <= 2 (k_qgemv): each wave on its own, activations straight from L2
//     into a three-deep (INT4) or four-deep (ternary) register ring with the
//     weights;
//   * 2 < B <= 32 (k_qgemv_wg): the four waves of a workgroup share one
//     superchunk range and its activations, staged in LDS.
#include "kans_common.h"
#include "kans_api_internal.h"
#include "kans_qgemv.h"
#include "kans_tile.h"
#include <algorithm>

namespace kans {

typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Re-tiling of the wire formats (run once per layer).
//
// Record order: one record per (row group of kQNW row blocks, superchunk),
// records of a row group consecutive in superchunk order, so each decode
// wave's superchunk range is one contiguous stream.  A record holds the kQNW
// code tiles (1 KB INT4 / 512 B ternary each) followed by their group
// parameters (kQNW x 16 rows x float4), see qrec_bytes.
// ---------------------------------------------------------------------------
template <int QT>
__host__ __device__ __forceinline__ long qrec_offset(int rb, int c, int C_tot) {
  return ((long)(rb / kQNW) * C_tot + c) * qrec_bytes(QT);
}
// byte offset of lane `lane`'s code word of row block rb, superchunk c (INT8:
// of its first 16 bytes; the second 16 follow 1 KB later, so that each of the
// tile's two 16-byte loads per lane reads 1 KB of whole cache lines)
template <int QT>
__host__ __device__ __forceinline__ long qcode_offset(int rb, int c, int C_tot, int lane) {
  if constexpr (QT == Q_TERN)  // row blocks 2p and 2p+1 paired: lane l's 16 bytes at 1 KB p + 16 l
    return qrec_offset<QT>(rb, c, C_tot) + (long)((rb % kQNW) >> 1) * 1024 + (long)lane * 16 + ((rb % kQNW) & 1) * 8;
  if constexpr (QT == Q_INT8)
    return qrec_offset<QT>(rb, c, C_tot) + (long)(rb % kQNW) * qtile_bytes(QT) + (long)lane * 16;
  return qrec_offset<QT>(rb, c, C_tot) + (long)(rb % kQNW) * qtile_bytes(QT) + (long)lane * (qtile_bytes(QT) / 64);
}
// code loads per record and lane (one 16-byte load per ternary tile pair)
__host__ __device__ constexpr int qcode_loads(int quant) {
  return quant == Q_INT8 ? 2 * kQNW : quant == Q_TERN ? kQNW / 2 : kQNW;
}
// byte offset of the group parameters (float4) of row r of row block rb, superchunk c
template <int QT>
__host__ __device__ __forceinline__ long qparam_offset(int rb, int c, int C_tot, int r) {
  return qrec_offset<QT>(rb, c, C_tot) + (long)kQNW * qtile_bytes(QT) + (long)((rb % kQNW) * 16 + r) * 16;
}

// INT4 qweight: row n is `rowbytes` bytes (groups of 64 nibbles contiguous,
// even index in the low nibble).  Q[rb][c][lane], lane = (q = l/16, r = l%16):
// dword t holds the 8 nibbles of row 16*rb + r at reduction indices
// 128c + 32t + 8q .. +7, i.e. bytes 64c + 16t + 4q .. +3 of the row.
__global__ void k_tile_int4(const unsigned char* __restrict__ qw, long rowbytes, int D_out, int nrb, int C,
                            int c_off, int C_tot, char* __restrict__ R) {
  const long total = (long)nrb * C * 64;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    const int lane = (int)(idx & 63);
    const long r2 = idx >> 6;
    const int c = (int)(r2 % C);
    const int rb = (int)(r2 / C);
    const int q = lane >> 4, r = lane & 15;
    const int n = rb * 16 + r;
    unsigned w[4] = {0u, 0u, 0u, 0u};
    if (n < D_out) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const long off = 64L * c + 16 * t + 4 * q;
        if (off < rowbytes) {
          const unsigned char* p = qw + (long)n * rowbytes + off;
          w[t] = (unsigned)p[0] | ((unsigned)p[1] << 8) | ((unsigned)p[2] << 16) | ((unsigned)p[3] << 24);
        }
      }
    }
    *reinterpret_cast<uint4*>(R + qcode_offset<Q_INT4>(rb, c_off + c, C_tot, lane)) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// INT8 qweight: row n is `rowbytes` bytes, one code per byte.  Q[rb][c][lane],
// lane = (q = l/16, r = l%16): dwords 2t, 2t+1 hold the 8 codes of row
// 16*rb + r at reduction indices 128c + 32t + 8q .. +7 (bytes of the row in
// order), i.e. 32 bytes per lane: dwords 0-3 at 16 l in the tile, dwords 4-7 at
// 1024 + 16 l (qcode_offset).
__global__ void k_tile_int8(const unsigned char* __restrict__ qw, long rowbytes, int D_out, int nrb, int C,
                            int c_off, int C_tot, char* __restrict__ R) {
  const long total = (long)nrb * C * 64;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    const int lane = (int)(idx & 63);
    const long r2 = idx >> 6;
    const int c = (int)(r2 % C);
    const int rb = (int)(r2 / C);
    const int q = lane >> 4, r = lane & 15;
    const int n = rb * 16 + r;
    unsigned w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    if (n < D_out) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const long off = 128L * c + 32 * t + 8 * q + 4 * hh;
          if (off < rowbytes) {
            const unsigned char* p = qw + (long)n * rowbytes + off;
            w[2 * t + hh] = (unsigned)p[0] | ((unsigned)p[1] << 8) | ((unsigned)p[2] << 16) | ((unsigned)p[3] << 24);
          }
        }
    }
    char* dst = R + qcode_offset<Q_INT8>(rb, c_off + c, C_tot, lane);
    *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    *reinterpret_cast<uint4*>(dst + 1024) = make_uint4(w[4], w[5], w[6], w[7]);
  }
}

// INT4 / INT8 group parameters: SB[rb][c][r] = (s0, s0', s1, s1') for the
// groups 2c, 2c+1 of row 16*rb + r, s' = b - 1024 s (zero past the row / matrix).
template <int QT>
__global__ void k_tile_affine_params(const float* __restrict__ scales, const float* __restrict__ biases, int gpr,
                                     int D_out, int nrb, int C, int c_off, int C_tot, char* __restrict__ R) {
  const long total = (long)nrb * C * 16;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    const int r = (int)(idx & 15);
    const long r2 = idx >> 4;
    const int c = (int)(r2 % C);
    const int rb = (int)(r2 / C);
    const int n = rb * 16 + r;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (n < D_out) {
#pragma unroll
      for (int gs = 0; gs < 2; ++gs) {
        const int g = 2 * c + gs;
        if (g < gpr) {
          const float s = scales[(long)n * gpr + g], b = biases[(long)n * gpr + g];
          v[2 * gs] = s;
          v[2 * gs + 1] = b - 1024.0f * s;
        }
      }
    }
    *reinterpret_cast<float4*>(R + qparam_offset<QT>(rb, c_off + c, C_tot, r)) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// Ternary w_packed: row n is `wpr` uint32 words, code of index j at bits
// 2*(j%16) of word j/16 (code 0 -> -1, 2 -> +1, 1 and 3 -> 0).
// T[rb][c][lane] (uint2; the words of row blocks 2p and 2p + 1 adjacent, so a
// lane loads both with one 16-byte load, qcode_offset; measured 2-3 % faster on
// the config-5 ternary block than one 8-byte load per row block): word u in
// {0,1} covers steps 2u and 2u+1; the 8 codes
// of step t for lane (q, r) are those of row 16*rb + r at indices
// j0 = 128c + 32t + 8q .. +7.  Each weight is stored as two bits, "non-zero"
// and "negative", placed so that the fp16 pair P = 4 (t & 1) + p (elements
// e = 2p, 2p + 1 of the step) is (word << kTernShift[P]) & 0x88008800: the
// non-zero bit lands on fp16 exponent bit 11, the sign on bit 15, so each
// element reads +-2^-13 or 0 (unpack_tern).  The eight shifts map the pairs
// onto disjoint bit sets that cover the word.
constexpr int kTernShift[8] = {11, 10, 9, 8, 3, 2, 1, 0};
constexpr unsigned kTernMask = 0x88008800u;

__device__ __forceinline__ unsigned tern_bits(unsigned code, int k, int half) {
  const unsigned nz = (code == 0u || code == 2u) ? 1u : 0u;
  const unsigned neg = code == 0u ? 1u : 0u;
  return (nz << (11 + 16 * half - k)) | (neg << (15 + 16 * half - k));
}

__global__ void k_tile_tern(const unsigned* __restrict__ wp, int wpr, long K_dim, int D_out, int nrb, int C,
                            int c_off, int C_tot, char* __restrict__ R) {
  const long total = (long)nrb * C * 64;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    const int lane = (int)(idx & 63);
    const long r2 = idx >> 6;
    const int c = (int)(r2 % C);
    const int rb = (int)(r2 / C);
    const int q = lane >> 4, r = lane & 15;
    const int n = rb * 16 + r;
    unsigned out[2] = {0u, 0u};
    if (n < D_out) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const long j0 = 128L * c + 32 * t + 8 * q;
        unsigned h = 0u;  // 8 codes, code e at bits 2e
        if (j0 < K_dim) {
          const unsigned word = wp[(long)n * wpr + j0 / 16];
          h = (word >> (2 * (j0 % 16))) & 0xffffu;
          const long valid = K_dim - j0;  // codes past K_dim read as 1 (zero weight)
          if (valid < 8) h = (h & ((1u << (2 * valid)) - 1u)) | (0x5555u & ~((1u << (2 * valid)) - 1u));
        } else {
          h = 0x5555u;
        }
        unsigned v = 0u;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const int k = kTernShift[4 * (t & 1) + p];
          v |= tern_bits((h >> (4 * p)) & 3u, k, 0);      // e = 2p
          v |= tern_bits((h >> (4 * p + 2)) & 3u, k, 1);  // e = 2p + 1
        }
        out[t >> 1] |= v;
      }
    }
    *reinterpret_cast<uint2*>(R + qcode_offset<Q_TERN>(rb, c_off + c, C_tot, lane)) = make_uint2(out[0], out[1]);
  }
}

// Ternary scales: SB[rb][c][r] = scales of the four 32-groups of superchunk c,
// times 2^13 (the unpacked weights are +-2^-13: every product phi * 2^-13 and
// every fp32 partial sum of them is exact scaling of the +-1 case, so
// (2^13 s) * g equals s * (2^13 g) bit for bit).
__global__ void k_tile_tern_params(const float* __restrict__ scales, int gpr, int D_out, int nrb, int C, int c_off,
                                   int C_tot, char* __restrict__ R) {
  const long total = (long)nrb * C * 16;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    const int r = (int)(idx & 15);
    const long r2 = idx >> 4;
    const int c = (int)(r2 % C);
    const int rb = (int)(r2 / C);
    const int n = rb * 16 + r;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (n < D_out) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int g = 4 * c + t;
        if (g < gpr) v[t] = scales[(long)n * gpr + g] * 8192.0f;
      }
    }
    *reinterpret_cast<float4*>(R + qparam_offset<Q_TERN>(rb, c_off + c, C_tot, r)) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// ---------------------------------------------------------------------------
// Activation basis.  Phi[m][p] (fp16, m < B of the MP allocated rows, p <
// C_tot*128; rows B .. MP-1 are not written, the GEMVs never store what they
// feed): the basis segment
// (p < Cb*128) holds T_k(clamp v[m][i]) at reduction index j = i*K + k, the base
// segment SiLU(v[m][i]) at j = i; within each 8-block the order is the unpack
// order pi of the weight format (INT4: 0,4,1,5,2,6,3,7; INT8 and ternary:
// identity).  S[c][m] = (sum over group 2c, sum over group 2c+1) of the
// fp16-rounded values (INT4 / INT8 only).  Indices past the segment's length
// are 0.
// ---------------------------------------------------------------------------
template <int QT>
__device__ __forceinline__ int unpack_order(int e) {
  if constexpr (QT == Q_INT4) return (e >> 1) + 4 * (e & 1);
  return e;
}

__device__ __forceinline__ float cheb_k(float t, int k) {
  // T_k(t) by the recurrence, as the reference (fused_kan.metal:216-236).
  float a = 1.0f, b = t;
  if (k == 0) return a;
  for (int i = 1; i < k; ++i) {
    const float c = __builtin_fmaf(2.0f * t, b, -a);
    a = b;
    b = c;
  }
  return b;
}

// SiLU with the reference's clip of the exponent argument (gated_kan.py:15-21).
__device__ __forceinline__ float silu_clip(float g) {
  const float c = fminf(fmaxf(g, -20.0f), 20.0f);
  return g / (1.0f + __expf(-c));
}

// fp32 -> 16-bit of a value first materialised in fp32.  Without the opaque
// register the compiler may fold the producing fma / multiply and the
// conversion into one v_fma_mixlo_f16 (a single rounding) in one kernel and
// not in another, and the decode kernels that must agree bit for bit
// (k_prep / k_qswiglu and the fused GEMV epilogues) would not.
__device__ __forceinline__ _Float16 half_of(float v) {
  asm volatile("" : "+v"(v));
  return (_Float16)v;
}
__device__ __forceinline__ float round16_of(float v, int mode) {
  asm volatile("" : "+v"(v));
  return mode == 2 ? to_f32(from_f32<__bf16>(v)) : (float)(_Float16)v;
}

__device__ __forceinline__ float load_any(const void* p, long i, int dt) {
  if (dt == DT_F32) return reinterpret_cast<const float*>(p)[i];
  if (dt == DT_F16) return (float)reinterpret_cast<const _Float16*>(p)[i];
  return to_f32(reinterpret_cast<const __bf16*>(p)[i]);
}

// Layer input v[m][i] of k_prep, and the layer's basis.
struct PrepIn {
  const void* X;
  int x_dtype;
  long ldx;
  int basis;       // BASIS_CHEBY / BASIS_RBF / BASIS_BSPLINE
  BasisParams bp;  // RBF / B-spline parameters
};

// Basis function k of the layer at input v, in fp32 (k_prep): Chebyshev T_k(clamp(v, -1, 1)) by the
// recurrence (fused_kan.metal:216-236); the Gaussian RBF exp(-(v - c_k)^2 inv_den) as
// exp2(neg_l (v - c_k)^2), neg_l = -inv_den log2(e) (fused_kan.metal:153-165); the clamped uniform
// cubic B-spline (fused_kan.metal:254-275, with the formulas of BasisGen<BASIS_BSPLINE>).
__device__ __forceinline__ float prep_basis(const PrepIn& in, float v, int k) {
  if (in.basis == BASIS_RBF) {
    const float d = v - in.bp.centers[k];
    return exp2f(in.bp.neg_l * (d * d));
  }
  if (in.basis == BASIS_BSPLINE) {
    const BasisParams& p = in.bp;
    const float pos = (v - p.grid_min) * p.inv_h;
    float fl = __builtin_floorf(pos);
    fl = __builtin_fminf(__builtin_fmaxf(fl, 0.0f), (float)(p.grid_size - 1));
    const float u = __builtin_fminf(__builtin_fmaxf(pos - fl, 0.0f), 1.0f);
    const int d = k - (int)fl;
    const float om = 1.0f - u, u2 = u * u, u3 = u2 * u, inv6 = 1.0f / 6.0f;
    if (d == 0) return om * om * om * inv6;
    if (d == 1) return (3.0f * u3 - 6.0f * u2 + 4.0f) * inv6;
    if (d == 2) return (-3.0f * u3 + 3.0f * u2 + 3.0f * u + 1.0f) * inv6;
    if (d == 3) return u3 * inv6;
    return 0.0f;
  }
  return cheb_k(fminf(fmaxf(v, -1.0f), 1.0f), k);
}

__device__ __forceinline__ float prep_input(const PrepIn& in, int m, int i) {
  return load_any(in.X, (long)m * in.ldx + i, in.x_dtype);
}

// One thread per (m, 8-block of the concatenated reduction axis).  Block = 256
// threads = 16 superchunks' worth of 8-blocks for one m (8-blocks of a
// superchunk are 16 consecutive threads, so group sums reduce within 8 lanes).
template <int QT>
__global__ void __launch_bounds__(256) k_prep(PrepIn in, int B, int MP, int D_in, int K, int has_base, int Cb,
                                              int C_tot, _Float16* __restrict__ Phi, float2* __restrict__ S) {
  const int m = blockIdx.y;
  const long blk = (long)blockIdx.x * 256 + threadIdx.x;  // 8-block index over C_tot*16
  const bool live = blk < (long)C_tot * 16;
  const long p0 = blk * 8;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = 0.0f;
  if (live && m < B) {
    const long Jb = (long)D_in * K;
    if (p0 < (long)Cb * 128) {
      // the 8 indices cover features i0 .. i0 + 8/K (+1); each input read once
      const long i0 = p0 / K;
      float xin[9];
      const int nf = (int)((p0 + 7) / K - i0) + 1;
#pragma unroll
      for (int f = 0; f < 9; ++f)
        if (f < nf && (i0 + f) * K < Jb) xin[f] = prep_input(in, m, (int)(i0 + f));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const long j = p0 + unpack_order<QT>(e);
        if (j < Jb) {
          const long i = j / K;
          v[e] = prep_basis(in, xin[i - i0], (int)(j - i * K));
        }
      }
    } else if (has_base) {
      const long i0 = p0 - (long)Cb * 128;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const long i = i0 + unpack_order<QT>(e);
        if (i < D_in) v[e] = silu_f32(prep_input(in, m, (int)i));
      }
    }
  }
  _Float16 hv[8];
  float sum = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    hv[e] = half_of(v[e]);
    sum += (float)hv[e];
  }
  if (live && m < MP) *reinterpret_cast<uint4*>(Phi + (long)m * C_tot * 128 + p0) = *reinterpret_cast<uint4*>(hv);
  if constexpr (q_affine(QT)) {
    // group of 64 = 8 consecutive 8-blocks = 8 consecutive lanes
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    sum += __shfl_xor(sum, 4);
    const float other = __shfl_xor(sum, 8);
    if (live && m < MP && (threadIdx.x & 15) == 0) S[(blk >> 4) * MP + m] = make_float2(sum, other);
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV.
// ---------------------------------------------------------------------------
// Unpack constants held in VGPRs: with two literal constants the compiler
// splits (a & mask) | orv into v_and + v_or (a VOP3 instruction here encodes no
// literal and reads at most one SGPR); as opaque register values it selects
// one v_and_or_b32.  The empty asm only hides the values from constant folding.
struct UnpackConsts {
  unsigned nib_mask, nib_magic, tern_mask, byte_magic;
  __device__ __forceinline__ void init() {
    nib_mask = 0x000F000Fu;
    nib_magic = 0x64006400u;
    tern_mask = kTernMask;
    byte_magic = 0x64646464u;  // high byte of fp16 1024 + q, for the INT8 v_perm_b32
    asm volatile("" : "+v"(nib_mask), "+v"(nib_magic), "+v"(tern_mask), "+v"(byte_magic));
  }
};

// INT4: 8 nibbles -> 8 fp16 values 1024+q in the order 0,4,1,5,2,6,3,7.
__device__ __forceinline__ half8v unpack_int4(unsigned w, const UnpackConsts& k) {
  unsigned o[4];
  o[0] = (w & k.nib_mask) | k.nib_magic;
  o[1] = ((w >> 4) & k.nib_mask) | k.nib_magic;
  o[2] = ((w >> 8) & k.nib_mask) | k.nib_magic;
  o[3] = ((w >> 12) & k.nib_mask) | k.nib_magic;
  return *reinterpret_cast<half8v*>(o);
}

// INT8: 8 bytes (two dwords, codes in order) -> 8 fp16 values 1024+q.
// v_perm_b32 selector bytes 0..3 pick bytes of the second operand (the codes),
// 4..7 bytes of the first (0x64): (q_e, 0x64, q_e+1, 0x64).
__device__ __forceinline__ half8v unpack_int8(unsigned w0, unsigned w1, const UnpackConsts& k) {
  unsigned o[4];
  o[0] = __builtin_amdgcn_perm(k.byte_magic, w0, 0x04010400u);
  o[1] = __builtin_amdgcn_perm(k.byte_magic, w0, 0x04030402u);
  o[2] = __builtin_amdgcn_perm(k.byte_magic, w1, 0x04010400u);
  o[3] = __builtin_amdgcn_perm(k.byte_magic, w1, 0x04030402u);
  return *reinterpret_cast<half8v*>(o);
}

// Ternary: the 8 weights of step 2u + B_STEP in word u (layout of k_tile_tern)
// -> 8 fp16 in {-2^-13, 0, +2^-13}: one shift and one AND per fp16 pair (the
// last pair of a word none), 15 instructions per 16 weights.
template <int B_STEP>
__device__ __forceinline__ half8v unpack_tern(unsigned w, const UnpackConsts& k) {
  unsigned o[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int sh = kTernShift[4 * B_STEP + p];
    o[p] = (sh ? (w << sh) : w) & k.tern_mask;
  }
  return *reinterpret_cast<half8v*>(o);
}

// One lane's code word of a tile (qtile_bytes / 64 bytes) and the B fragment
// of MFMA step t (reduction indices 32t .. 32t + 31 of the superchunk) in it.
struct QW8 {
  uint4 lo, hi;
};
template <int QT>
using QWordOf = typename std::conditional<QT == Q_INT4, uint4,
                                          typename std::conditional<QT == Q_INT8, QW8, uint2>::type>::type;
template <int QT, int T, typename QW>
__device__ __forceinline__ half8v unpack_step(const QW& qw, const UnpackConsts& k) {
  const unsigned* dw = reinterpret_cast<const unsigned*>(&qw);
  if constexpr (QT == Q_INT4) return unpack_int4(dw[T], k);
  else if constexpr (QT == Q_INT8) return unpack_int8(dw[2 * T], dw[2 * T + 1], k);
  else return unpack_tern<T & 1>(dw[T >> 1], k);
}

struct QMatDev {
  const char* rec;      // records [nrb_pad / kQNW][C_tot], qrec_bytes each
  int D_out;
  int col_off;          // column offset of this matrix in the output / workspace
};

// ---------------------------------------------------------------------------
// Fused epilogue (QEpi).  The partial sums of the fused launches are written
// with agent-scope atomic stores and read back with agent-scope atomic loads;
// an arrival counter picks the wave that reduces them.  The ordering argument
// is at the ISA level (gfx942 / gfx950 memory model as LLVM implements it,
// AMDGPUUsage "Memory Model GFX942"):
//   * an agent-scope atomic store is `global_store ... sc1`: it is written
//     through the XCD's L2 to the memory-side coherence point, and its
//     vector-memory counter decrement (vmcnt) comes with that write's
//     acknowledgement;
//   * an agent-scope atomic load is `global_load ... sc1`: it does not hit a
//     non-coherent L2 line, so it reads the coherence point;
//   * each wave waits `s_waitcnt vmcnt(0)` (all of its partial stores
//     acknowledged) before its counter RMW, which is performed at the
//     coherence point; the last arriver issues its partial loads only after
//     its RMW returned (the loads depend on the returned value, and a second
//     vmcnt(0) precedes them).
// So every partial store is visible before any partial load of the reduction
// is issued.  The C++-level alternative (agent-scope release on the RMW and an
// acquire fence in the last arriver) compiles to `buffer_wbl2 sc1` in every
// arriving wave and `buffer_inv sc1` in the last one, and measured 143 us
// instead of 85 us for the config-5 INT4 block at B = 1 (the L2 write-back
// and invalidation of ~1700 waves); the bitwise fused-vs-separate-kernel test
// (test_gated_fused_epilogue_matches_unfused) checks the result.
// ---------------------------------------------------------------------------
constexpr int kWaitVmem = 0 | (0x7 << 4) | (0xf << 8);  // s_waitcnt vmcnt(0) only

__device__ __forceinline__ void part_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float part_load(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Counts this wave's arrival at counter *c; true for the last of `need`
// arrivals, which also resets the counter for the next launch.  Every wave of
// the group arrives exactly once per launch and none waits for another.  The
// reset needs no ordering of its own: the next launch starts after this one
// has ended (same stream).
__device__ __forceinline__ bool last_arrival(int* c, int need, int lane) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(kWaitVmem);  // this wave's partial stores are acknowledged
  int old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __shfl(old, 0);
  if (old != need - 1) return false;
  __builtin_amdgcn_s_waitcnt(kWaitVmem);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  if (lane == 0) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// Writes 8-blocks [b_lo, b_hi) of one Phi row from the staged values st (local
// index i < n_st; 0 past it), index p0 = p_lo + 8b, in the unpack order of the
// weight format; INT4 also writes the group sums of the fp16 values (groups of
// 64 = 8 blocks, summed as k_prep does).
template <int QT>
__device__ __forceinline__ void epi_write_blocks(const _Float16* st, int n_st, long p_lo, int nblk, _Float16* phi_row,
                                                 float* S2f, int MP, int m, int lane) {
  for (int b0 = 0; b0 < nblk; b0 += 64) {
    const int b = b0 + lane;
    const bool live = b < nblk;
    _Float16 hv[8];
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = 8 * b + unpack_order<QT>(e);
      hv[e] = live && i < n_st ? st[i] : (_Float16)0.0f;
      sum += (float)hv[e];
    }
    const long p0 = p_lo + 8L * b;
    if (live) *reinterpret_cast<uint4*>(phi_row + p0) = *reinterpret_cast<uint4*>(hv);
    if constexpr (q_affine(QT)) {
      sum += __shfl_xor(sum, 1);
      sum += __shfl_xor(sum, 2);
      sum += __shfl_xor(sum, 4);
      if (live && (b & 7) == 0) {
        const long G = p0 >> 6;
        S2f[((G >> 1) * MP + m) * 2 + (G & 1)] = sum;
      }
    }
  }
}

// QEPI_SWIGLU for feature group j (lane = feature 64j + lane): hidden as
// k_qswiglu (same sum order and rounding), then T_k(clamp(hidden)) and
// SiLU(hidden) into the next layer's Phi / S as k_prep.  The group covering
// the last features also writes the zero padding up to each segment's end.
// Rows m_lo .. m_hi - 1; AT: read the partial sums with agent-scope loads
// (written by other waves of the same launch), else plain loads (written by an
// earlier launch).
template <int QT, bool AT>
__device__ __forceinline__ void epi_swiglu(const QEpi& E, const float* part, int ksplit, int B, int MP, int h, int j,
                                           int n_groups, _Float16* st, int lane, int m_lo, int m_hi) {
  const int f = j * 64 + lane;
  const int K2 = E.K2;
  const long total = (long)B * 2 * h;
  const long ldphi2 = (long)E.C_tot2 * 128;
  const bool last = j == n_groups - 1;
  const long pb_lo = (long)j * 64 * K2;
  const long pb_hi = last ? (long)E.Cb2 * 128 : pb_lo + 64L * K2;
  const long pw_lo = (long)E.Cb2 * 128 + 64L * j;
  const long pw_hi = last ? ldphi2 : pw_lo + 64;
  float* S2f = reinterpret_cast<float*>(E.S2);
  for (int m = m_lo; m < m_hi; ++m) {
    float hvv = 0.0f;
    if (f < h) {
      float g = E.bias ? load_any(E.bias, f, E.bias_dtype) : 0.0f;
      float u = E.bias_u ? load_any(E.bias_u, f, E.bias_u_dtype) : 0.0f;
      const float* p = part + (long)m * 2 * h + f;
      for (int k0 = 0; k0 < ksplit; k0 += 8) {
        float vg[8], vu[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const float* pg = p + (long)(k0 + q) * total;
          vg[q] = k0 + q < ksplit ? (AT ? part_load(pg) : *pg) : 0.f;
          vu[q] = k0 + q < ksplit ? (AT ? part_load(pg + h) : pg[h]) : 0.f;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (k0 + q < ksplit) {
            g += vg[q];
            u += vu[q];
          }
      }
      if (E.round16) {
        g = round16_of(g, E.round16);
        u = round16_of(u, E.round16);
      }
      hvv = silu_clip(g) * u;
      if (E.round16) hvv = round16_of(hvv, E.round16);
    }
    // stage T_0 .. T_{K2-1} at lane*K2 + k and SiLU at 64*K2 + lane (0 past h)
    const float t = fminf(fmaxf(hvv, -1.0f), 1.0f);
    float a = 1.0f, bb = t;
    for (int k = 0; k < K2; ++k) {
      float v = k == 0 ? a : bb;
      if (k >= 2) {
        const float c = __builtin_fmaf(2.0f * t, bb, -a);
        a = bb;
        bb = c;
        v = c;
      }
      st[lane * K2 + k] = f < h ? half_of(v) : (_Float16)0.0f;
    }
    st[64 * K2 + lane] = f < h && E.has_base2 ? half_of(silu_f32(hvv)) : (_Float16)0.0f;
    asm volatile("" ::: "memory");  // LDS writes before the reads below (one wave, in order)
    _Float16* row = E.Phi2 + (long)m * ldphi2;
    epi_write_blocks<QT>(st, 64 * K2, pb_lo, (int)((pb_hi - pb_lo) / 8), row, S2f, MP, m, lane);
    if (E.has_base2) epi_write_blocks<QT>(st + 64 * K2, 64, pw_lo, (int)((pw_hi - pw_lo) / 8), row, S2f, MP, m, lane);
    asm volatile("" ::: "memory");  // reads done before the next row's writes
  }
}

// Load of one 8- or 16-byte word of a weight record: plain, or non-temporal
// (NT: the caches are told the data is streamed once).  Non-temporal loads
// leave L2 and the MALL to other data and stream faster when the weights
// cannot stay cached between calls anyway (more than the MALL holds); plain
// loads let a block whose weights fit the MALL hit it on the next call.
template <bool NT, typename Q>
__device__ __forceinline__ Q load_rec(const char* p) {
  if constexpr (sizeof(Q) == 32) {
    Q q;
    q.lo = load_rec<NT, uint4>(p);
    q.hi = load_rec<NT, uint4>(p + 16);
    return q;
  } else if constexpr (!NT) {
    return *reinterpret_cast<const Q*>(p);
  } else {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    static_assert(sizeof(Q) == 16 || sizeof(Q) == 8, "8- or 16-byte words");
    Q q;
    if constexpr (sizeof(Q) == 16) {
      const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
      __builtin_memcpy(&q, &v, 16);
    } else {
      const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
      __builtin_memcpy(&q, &v, 8);
    }
    return q;
  }
}

// The kQNW code words of one record for this lane (layout of qcode_offset).
// rec is wave-uniform and the lane's offset an unsigned 32-bit value, so each
// load can take the scalar-base + vector-offset form (no 64-bit address in
// vector registers that the compiler could reuse as the load's destination).
template <bool NT, int QT, typename QW>
__device__ __forceinline__ void load_codes(const char* rec, int lane, QW (&qw)[kQNW]) {
  const unsigned lo = (unsigned)lane * 16u;
  if constexpr (QT == Q_TERN) {
#pragma unroll
    for (int p = 0; p < kQNW / 2; ++p) {
      const uint4 v = load_rec<NT, uint4>(rec + p * 1024 + lo);
      qw[2 * p] = make_uint2(v.x, v.y);
      qw[2 * p + 1] = make_uint2(v.z, v.w);
    }
  } else if constexpr (QT == Q_INT8) {
    // the two halves of the lane's 32 bytes, 1 KB apart (qcode_offset)
#pragma unroll
    for (int w = 0; w < kQNW; ++w) {
      qw[w].lo = load_rec<NT, uint4>(rec + w * qtile_bytes(QT) + lo);
      qw[w].hi = load_rec<NT, uint4>(rec + w * qtile_bytes(QT) + 1024 + lo);
    }
  } else {
    static_assert(sizeof(QW) == 16, "INT4 code words: 16 bytes per lane");
#pragma unroll
    for (int w = 0; w < kQNW; ++w) qw[w] = load_rec<NT, QW>(rec + w * qtile_bytes(QT) + lo);
  }
}

// The same loads through a buffer resource over the wave's row group of
// records (k_qgemv): the lane's offset is one loop-invariant vector register and
// the record's offset a scalar, so no 64-bit address is rebuilt in vector
// registers for every superchunk (with pointer loads the compiler made one
// load's address registers its destination, and the ring loop then waited for
// every load in flight before it could rebuild the next address).
__device__ __forceinline__ uint4 load_buf16(__amdgpu_buffer_rsrc_t r, unsigned voff, int soff, bool nt) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = nt ? __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2)
                     : __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
template <bool NT, int QT, typename QW>
__device__ __forceinline__ void load_codes_buf(__amdgpu_buffer_rsrc_t r, int soff, int lane, QW (&qw)[kQNW]) {
  const unsigned lo = (unsigned)lane * 16u;
  if constexpr (QT == Q_TERN) {
#pragma unroll
    for (int p = 0; p < kQNW / 2; ++p) {
      const uint4 v = load_buf16(r, lo + p * 1024, soff, NT);
      qw[2 * p] = make_uint2(v.x, v.y);
      qw[2 * p + 1] = make_uint2(v.z, v.w);
    }
  } else if constexpr (QT == Q_INT8) {
#pragma unroll
    for (int w = 0; w < kQNW; ++w) {
      qw[w].lo = load_buf16(r, lo + w * qtile_bytes(QT), soff, NT);
      qw[w].hi = load_buf16(r, lo + w * qtile_bytes(QT) + 1024, soff, NT);
    }
  } else {
#pragma unroll
    for (int w = 0; w < kQNW; ++w) qw[w] = load_buf16(r, lo + w * qtile_bytes(QT), soff, NT);
  }
}

// In-kernel activation basis of k_qgemv (PRE): the layer input and the basis
// geometry, and the workgroup's LDS slice: Phi rows [SR][span * 128] (fp16, in
// the weight format's unpack order) then the group sums [span][SR] (INT4 / INT8).
struct QPreDev {
  const void* X;
  int x_dtype;
  long ldx;
  int D_in, K, has_base, Cb;
  int span;   // superchunks per slice, >= every workgroup's range
  int slice;  // bytes of the workgroup's LDS slice (the waves' epilogue stages follow it)
};
constexpr int kPreThreads = 256;       // threads of a workgroup computing one range's basis together
constexpr int kEpiStageBytes = 64 * (kMaxK + 1) * 2;  // a wave's SwiGLU epilogue stage (fp16)
constexpr int kPreBatch = 4;            // input loads in flight per thread
constexpr int kPreVec = 2;              // 16-byte input loads in flight per thread (base segment)
constexpr int kPreLdsMax = 80 * 1024;   // dynamic LDS per workgroup (two per CU)

// One batch of layer inputs, x[m][min(fb + pt + kPreThreads it, f1 - 1)] for
// it < kPreBatch, as raw bits (4- or 2-byte loads under one uniform branch):
// no value is used before the batch's last load is issued, so the loads stay
// in flight together (converted in the branch, each load was waited for in
// turn).  x_of_raw converts as load_any does (all three conversions exact).
__device__ __forceinline__ void load_x_raw(unsigned (&xr)[kPreBatch], const QPreDev& P, int m, int fb, int f1,
                                           int pt) {
  // a uniform row pointer and 32-bit lane offsets: one VGPR per address
  const int es = P.x_dtype == DT_F32 ? 4 : 2;
  const char* row = reinterpret_cast<const char*>(P.X) + (long)m * P.ldx * es;
  if (es == 4) {
#pragma unroll
    for (int it = 0; it < kPreBatch; ++it)
      xr[it] = *reinterpret_cast<const unsigned*>(row + 4u * (unsigned)min(fb + pt + kPreThreads * it, f1 - 1));
  } else {
#pragma unroll
    for (int it = 0; it < kPreBatch; ++it)
      xr[it] = *reinterpret_cast<const unsigned short*>(row + 2u * (unsigned)min(fb + pt + kPreThreads * it, f1 - 1));
  }
}
__device__ __forceinline__ float x_of_raw(unsigned r, int dt) {
  if (dt == DT_F32) return __uint_as_float(r);
  if (dt == DT_F16) return (float)__builtin_bit_cast(_Float16, (unsigned short)r);
  return __uint_as_float(r << 16);  // bf16
}

// LDS / Phi position of reduction index rp within its 8-block: the inverse of
// unpack_order.
template <int QT>
__device__ __forceinline__ int unpack_pos(int rp) {
  if constexpr (QT == Q_INT4) {
    const int u = rp & 7;
    return (rp & ~7) | (u < 4 ? 2 * u : 2 * (u - 4) + 1);
  }
  return rp;
}

// In-kernel basis of x, Chebyshev with K = 4 or 8 coefficients: the 8-blocks
// b < nblocks of a workgroup's range (reduction indices P_lo + 8 b .. + 7, all
// in the basis segment), one per thread pt and step.  A block covers 8 / K
// whole features; the thread evaluates T_0 .. T_{K-1} of them with k_prep's
// recurrence (cheb_k: the same fma chain, so the same values), converts them
// with half_of, places them in the weight format's unpack order and writes the
// block with one 16-byte LDS store.  The input loads of a step are issued
// together, then kick() (the wave's first weight loads), then the arithmetic.
// The per-value form (below) spent ~8 us per wave at cfg5 in its 64-bit index
// arithmetic and 2-byte LDS stores; this form writes whole blocks.
constexpr int kPreBlocks = 2;    // 8-blocks per thread and step
template <int QT, int KC, typename Kick>
__device__ __forceinline__ void pre_cheb_blocks(const QPreDev& P, int m, long P_lo, int nblocks, _Float16* dst,
                                                int pt, Kick&& kick) {
  constexpr int NF = 8 / KC;  // features per block
  const int es = P.x_dtype == DT_F32 ? 4 : 2;
  const char* row = reinterpret_cast<const char*>(P.X) + (long)m * P.ldx * es;
  const unsigned f_base = (unsigned)(P_lo / KC);  // feature of block 0's first index (P_lo is a multiple of 128)
  for (int b0 = 0; b0 < nblocks; b0 += kPreThreads * kPreBlocks) {
    unsigned xr[kPreBlocks][NF];
    if (es == 4) {
#pragma unroll
      for (int it = 0; it < kPreBlocks; ++it) {
        const unsigned f = f_base + (unsigned)min(b0 + pt + kPreThreads * it, nblocks - 1) * NF;
#pragma unroll
        for (int q = 0; q < NF; ++q) xr[it][q] = *reinterpret_cast<const unsigned*>(row + 4u * (f + q));
      }
    } else {
#pragma unroll
      for (int it = 0; it < kPreBlocks; ++it) {
        const unsigned f = f_base + (unsigned)min(b0 + pt + kPreThreads * it, nblocks - 1) * NF;
#pragma unroll
        for (int q = 0; q < NF; ++q) xr[it][q] = *reinterpret_cast<const unsigned short*>(row + 2u * (f + q));
      }
    }
    kick();
#pragma unroll
    for (int it = 0; it < kPreBlocks; ++it) {
      const int b = b0 + pt + kPreThreads * it;
      if (b < nblocks) {
        float T[NF][KC];
#pragma unroll
        for (int q = 0; q < NF; ++q) {
          const float t = fminf(fmaxf(x_of_raw(xr[it][q], P.x_dtype), -1.0f), 1.0f);
          T[q][0] = 1.0f;
          T[q][1] = t;
#pragma unroll
          for (int k = 2; k < KC; ++k) T[q][k] = __builtin_fmaf(2.0f * t, T[q][k - 1], -T[q][k - 2]);
        }
        // position e holds index unpack_order(e) of the block: feature u / KC, coefficient u % KC
        _Float16 hv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int u = unpack_order<QT>(e);
          hv[e] = half_of(T[u / KC][u % KC]);
        }
        reinterpret_cast<uint4*>(dst)[b] = *reinterpret_cast<const uint4*>(hv);
      }
    }
  }
}

// Small-batch decode GEMV (B = SR <= kSmallB).  One wave = kQNW row blocks
// (64 output rows) x one contiguous superchunk range (split-K over waves for
// memory-level parallelism); 4 independent waves per workgroup.
// part[ks][m][col] (m < B) receives the wave's partial sums.
//
// The activation fragment carries batch row m in MFMA rows m, 4 + m, 8 + m
// and 12 + m, so every lane group q = 0..3 receives all SR live rows in
// accumulator registers 0..SR-1, and lane (q, r) finishes row block q of the
// wave: one full-wave 16-byte load brings each lane the group parameters of
// its own row (row block q, row r) and the epilogue applies them to every tile
// (only tile q's result is kept and stored).  The parameters cost 4 registers
// per superchunk in flight instead of 16, and one load instruction instead of
// four.  Lanes whose MFMA row is not a batch row load batch row 0's fragment
// (the same cache line as its own lanes): their results only reach
// accumulator rows that are not stored, and an unconditional load keeps the
// loop free of branches (with the load under a branch, the compiler's wait
// counts merged across it and it drained the ring at every round; it also
// held ~90 more registers).  NT: non-temporal weight loads (load_rec).
//
// PRE: the four waves of a workgroup take four consecutive row groups over
// one superchunk range, and its 256 threads compute Phi / S of that range from
// the layer input into the workgroup's LDS slice first (QPreDev), with the
// values, rounding and sum order of k_prep, so the results equal the k_prep
// path bit for bit; two barriers order the basis values, the sums and the
// reads.  Each wave's first weight loads are issued right after the first
// batch of input loads, so the inputs return first and the weights stream
// while the basis is computed; the k_prep launch and its wait disappear.
// (Each wave computing its own range's basis alone spent 5-16 us per wave on
// it at cfg5, a quarter of the gate|up GEMV's time.)
template <int QT, int SR, int EPI, bool NT, bool PRE>
__global__ void __launch_bounds__(256) k_qgemv(QMatDev m0, QMatDev m1, int rg_split, int n_rg, int ksplit,
                                               int C_tot, const _Float16* __restrict__ Phi,
                                               const float2* __restrict__ S, int B, int MP,
                                               float* __restrict__ part, int N_total, QEpi E, QPreDev P) {
  static_assert(SR >= 1 && SR <= kSmallB, "small-batch kernel");
  constexpr int NW = kQNW;
  const int lane = threadIdx.x & 63;
  // the wave index as a scalar: record bases, ranges and row groups are then
  // wave-uniform, and the weight loads take the scalar-base + lane-offset form
  // (with the base in vector registers the compiler reused a load's address
  // registers as its destination, and the next round's address then waited for
  // every load in flight at the top of the ring loop)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // PRE: the four waves of a workgroup take four consecutive row groups over
  // ONE superchunk range and compute its basis together (a workgroup past the
  // last row group still takes part in that, then stops); otherwise four
  // consecutive (row group, split) items
  const int item = blockIdx.x * 4 + wave;
  const int rg_all = PRE ? (int)(blockIdx.x / ksplit) * 4 + wave : item / ksplit;
  const int ks = PRE ? (int)(blockIdx.x % ksplit) : item - rg_all * ksplit;
  const bool live_rg = rg_all < n_rg;
  if (!PRE && !live_rg) return;  // uniform per wave
  const int rg = live_rg ? rg_all : n_rg - 1;
  const QMatDev& M = rg < rg_split ? m0 : m1;
  const int rg_loc = rg < rg_split ? rg : rg - rg_split;
  const int rb0 = rg_loc * NW;
  const int c_lo = (int)((long)C_tot * ks / ksplit);
  const int c_hi = (int)((long)C_tot * (ks + 1) / ksplit);
  const int q = lane >> 4, r = lane & 15;
  const long ldphi = (long)C_tot * 128;
  UnpackConsts uk;
  uk.init();

  floatx4 acc[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) acc[w] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int arow = r & 3;  // batch row of this lane's MFMA row (replicated every 4 rows)
  const bool alive = arow < B;
  const _Float16* arow_p = Phi + (long)(alive ? arow : 0) * ldphi + 8 * q;
  // PRE: the workgroup's LDS slice (basis values, then group sums), then one
  // epilogue stage per wave
  extern __shared__ __attribute__((aligned(16))) char qg_dyn[];
  const int pt = threadIdx.x;  // thread of the workgroup in the basis work
  _Float16* const phl = reinterpret_cast<_Float16*>(qg_dyn);
  float2* const sl = reinterpret_cast<float2*>(qg_dyn + P.span * SR * 256);
  const int lrow = P.span * 128;
  const _Float16* const arow_l = phl + (alive ? arow : 0) * lrow + 8 * q;

  typedef QWordOf<QT> QWord;
  const char* rbase = M.rec + (long)rg_loc * C_tot * qrec_bytes(QT);
  // this row group's records (C_tot of them) as one buffer (see load_codes_buf)
  const __amdgpu_buffer_rsrc_t rrec =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(rbase), (short)0, C_tot * qrec_bytes(QT), 0x00020000);

  // operands of one superchunk: weights / group parameters (HBM stream) and
  // activation fragments / group sums (L2 resident).
  struct Ops {
    QWord qw[NW];
    float4 sb;        // this lane's own row (row block q, row r)
    half8v a[4];
    float2 sg[SR];    // INT4 / INT8: group sums of batch rows 0 .. SR-1 (the same in every lane)
  };
  auto compute = [&](const Ops& o) {
    if constexpr (q_affine(QT)) {
      static_for<0, 2>([&](auto GS) __attribute__((always_inline)) {
        constexpr int gs = decltype(GS)::value;
        floatx4 g[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const half8v b0 = unpack_step<QT, 2 * gs>(o.qw[w], uk);
          const half8v b1 = unpack_step<QT, 2 * gs + 1>(o.qw[w], uk);
          g[w] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.a[2 * gs], b0, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          g[w] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.a[2 * gs + 1], b1, g[w], 0, 0, 0);
        }
        const float s = gs ? o.sb.z : o.sb.x;
        const float s2 = gs ? o.sb.w : o.sb.y;
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
          for (int i = 0; i < SR; ++i) {
            const float S_ = gs ? o.sg[i].y : o.sg[i].x;
            acc[w][i] = __builtin_fmaf(s, g[w][i], __builtin_fmaf(s2, S_, acc[w][i]));
          }
      });
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        floatx4 g[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const unsigned* dw = reinterpret_cast<const unsigned*>(&o.qw[w]);
          const half8v bf = (t & 1) ? unpack_tern<1>(dw[t >> 1], uk) : unpack_tern<0>(dw[t >> 1], uk);
          g[w] = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.a[t], bf, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
        const float s = t == 0 ? o.sb.x : t == 1 ? o.sb.y : t == 2 ? o.sb.z : o.sb.w;
#pragma unroll
        for (int w = 0; w < NW; ++w)
#pragma unroll
          for (int i = 0; i < SR; ++i) acc[w][i] = __builtin_fmaf(s, g[w][i], acc[w][i]);
      }
    }
  };

  if (c_lo < c_hi) {
    // Register ring: superchunks c+1 and c+2 are in flight while c is
    // consumed (INT4 ~10 KB per wave).  Loads past the end of the range
    // repeat the last superchunk (an L2 hit, no extra HBM traffic), so the
    // loop body is branch-free and compute(c) waits for exactly the operands
    // of c (vmcnt counts in issue order).  A four-deep ring for ternary, whose
    // records are half the size, measured slower with this loop (cfg5 block
    // at B = 1: 73.2 against 69.2 us).
    // RD slots, superchunks c+1 .. c+RD-1 in flight while c is consumed
    constexpr int RD = qring_depth(QT);
    Ops o[RD];
    // activation fragments and group sums of superchunk c: from Phi / S, or
    // (PRE) from the wave's LDS slice
    auto issue_a = [&](int c, Ops& o) {
      const int cc = min(c, c_hi - 1);
      if constexpr (PRE) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          o.a[t] = *reinterpret_cast<const half8v*>(arow_l + (cc - c_lo) * 128 + 32 * t);
        if constexpr (q_affine(QT)) {
#pragma unroll
          for (int i = 0; i < SR; ++i) o.sg[i] = sl[(cc - c_lo) * SR + i];
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          o.a[t] = *reinterpret_cast<const half8v*>(arow_p + (long)cc * 128 + 32 * t);
        if constexpr (q_affine(QT)) {
#pragma unroll
          for (int i = 0; i < SR; ++i) o.sg[i] = S[(long)cc * MP + i];
        }
      }
    };
    auto issue_w = [&](int c, Ops& o) {
      const int soff = min(c, c_hi - 1) * qrec_bytes(QT);
      load_codes_buf<NT, QT>(rrec, soff, lane, o.qw);
      const uint4 sb = load_buf16(rrec, (unsigned)lane * 16u + NW * qtile_bytes(QT), soff, NT);
      o.sb = make_float4(__uint_as_float(sb.x), __uint_as_float(sb.y), __uint_as_float(sb.z), __uint_as_float(sb.w));
    };
    auto issue = [&](int c, Ops& o) {
      issue_a(c, o);
      issue_w(c, o);
    };
    // The loop body is whole rounds of three superchunks with no exit
    // inside: with an exit per superchunk the compiler's wait counts merged
    // across the exits and it drained the ring (vmcnt(0)) at the top of every
    // round.  Scheduling fences before each issue keep one superchunk's loads
    // together and the slots in ring order.
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
    if constexpr (PRE) {
      bool started = false;
      // the ring's first weight loads, issued once, right after the first
      // batch of input loads
      auto kick = [&] {
        if (started || !live_rg) return;
        started = true;
        static_for<0, RD - 1>([&](auto J) __attribute__((always_inline)) {
          fence();
          issue_w(c_lo + decltype(J)::value, o[decltype(J)::value]);
        });
        fence();
      };
      const long P_lo = (long)c_lo * 128, P_hi = (long)c_hi * 128;
      const int nblk = (c_hi - c_lo) * 16;
      // zero the slice: indices past the segments' values read 0
#pragma unroll
      for (int m = 0; m < SR; ++m)
        for (int i = pt; i < nblk; i += kPreThreads)
          reinterpret_cast<uint4*>(phl + m * lrow)[i] = make_uint4(0u, 0u, 0u, 0u);
      // basis segment: T_k(clamp(x_i)) at index i K + k (k_prep / cheb_k)
      const long Pb_end = min(P_hi, min((long)P.Cb * 128, (long)P.D_in * P.K));
      // K = 4 and 8: whole 8-blocks per lane (pre_cheb_blocks), the rest per feature below
      long Pg_lo = P_lo;
      if (P_lo < Pb_end && (P.K == 4 || P.K == 8)) {
        const int nfull = (int)((Pb_end - P_lo) / 8);
        for (int m = 0; m < SR; ++m) {
          if (P.K == 4) pre_cheb_blocks<QT, 4>(P, m, P_lo, nfull, phl + m * lrow, pt, kick);
          else pre_cheb_blocks<QT, 8>(P, m, P_lo, nfull, phl + m * lrow, pt, kick);
        }
        Pg_lo = P_lo + 8L * nfull;
      }
      if (Pg_lo < Pb_end) {
        const int f0 = (int)(Pg_lo / P.K), f1 = (int)((Pb_end - 1) / P.K) + 1;
        for (int m = 0; m < SR; ++m)
          for (int fb = f0; fb < f1; fb += kPreThreads * kPreBatch) {
            unsigned xr[kPreBatch];
            load_x_raw(xr, P, m, fb, f1, pt);
            kick();
#pragma unroll
            for (int it = 0; it < kPreBatch; ++it) {
              const int f = fb + pt + kPreThreads * it;
              if (f < f1) {
                const float t = fminf(fmaxf(x_of_raw(xr[it], P.x_dtype), -1.0f), 1.0f);
                float a = 1.0f, b = t;
                for (int k = 0; k < P.K; ++k) {
                  float v = k == 0 ? a : b;
                  if (k >= 2) {
                    const float cn = __builtin_fmaf(2.0f * t, b, -a);
                    a = b;
                    b = cn;
                    v = cn;
                  }
                  const long j = (long)f * P.K + k;
                  if (j >= Pg_lo && j < Pb_end) phl[m * lrow + unpack_pos<QT>((int)(j - P_lo))] = half_of(v);
                }
              }
            }
          }
      }
      // base segment: SiLU(x_i) at index Cb * 128 + i
      if (P.has_base) {
        const long w0 = (long)P.Cb * 128;
        const long Pw0 = max(P_lo, w0), Pw1 = min(P_hi, w0 + P.D_in);
        const int es = P.x_dtype == DT_F32 ? 4 : 2;
        // 16-byte loads of 8 consecutive inputs when the rows allow them:
        // one 8-block per load, so a whole base range is one batch
        const bool vec = (P.D_in & 7) == 0 &&
                         ((reinterpret_cast<unsigned long>(P.X) | (unsigned long)(P.ldx * es)) & 15) == 0;
        if (Pw0 < Pw1 && vec) {
          const int ch0 = (int)(Pw0 - w0) / 8, ch1 = (int)(Pw1 - w0) / 8;  // 8-input chunks
          for (int m = 0; m < SR; ++m) {
            const char* row = reinterpret_cast<const char*>(P.X) + (long)m * P.ldx * es;
            // chunks per thread and step: kPreVec (16-bit x, one load each) or
            // kPreVec / 2 (fp32 x, two loads each)
            const int cstep = kPreThreads * (es == 2 ? kPreVec : kPreVec / 2);
            for (int cb = ch0; cb < ch1; cb += cstep) {
              uint4 xr[kPreVec];  // es = 2: one chunk each; es = 4: half a chunk each
              if (es == 2) {
#pragma unroll
                for (int it = 0; it < kPreVec; ++it)
                  xr[it] = *reinterpret_cast<const uint4*>(
                      row + 16u * (unsigned)min(cb + pt + kPreThreads * it, ch1 - 1));
              } else {
#pragma unroll
                for (int it = 0; it < kPreVec; ++it)
                  xr[it] = *reinterpret_cast<const uint4*>(
                      row + 32u * (unsigned)min(cb + pt + kPreThreads * (it >> 1), ch1 - 1) + 16u * (unsigned)(it & 1));
              }
              kick();
              // chunk `it` of this thread: SiLU of its 8 inputs into one 8-block
              auto put = [&](int it, const float (&v)[8]) {
                const int ch = cb + pt + kPreThreads * it;
                if (ch < ch1) {
                  _Float16 hv[8];
#pragma unroll
                  for (int e = 0; e < 8; ++e) hv[e] = half_of(silu_f32(v[unpack_order<QT>(e)]));
                  *reinterpret_cast<uint4*>(phl + m * lrow + (w0 + 8L * ch - P_lo)) = *reinterpret_cast<uint4*>(hv);
                }
              };
              if (es == 2) {
#pragma unroll
                for (int it = 0; it < kPreVec; ++it) {
                  const unsigned* w = reinterpret_cast<const unsigned*>(&xr[it]);
                  float v[8];
#pragma unroll
                  for (int e = 0; e < 8; ++e) v[e] = x_of_raw((w[e >> 1] >> (16 * (e & 1))) & 0xffffu, P.x_dtype);
                  put(it, v);
                }
              } else {
#pragma unroll
                for (int it = 0; it < kPreVec / 2; ++it) {
                  const unsigned* w0p = reinterpret_cast<const unsigned*>(&xr[2 * it]);
                  const unsigned* w1p = reinterpret_cast<const unsigned*>(&xr[2 * it + 1]);
                  float v[8];
#pragma unroll
                  for (int e = 0; e < 4; ++e) {
                    v[e] = __uint_as_float(w0p[e]);
                    v[4 + e] = __uint_as_float(w1p[e]);
                  }
                  put(it, v);
                }
              }
            }
          }
        } else if (Pw0 < Pw1) {
          const int f0 = (int)(Pw0 - w0), f1 = (int)(Pw1 - w0);
          for (int m = 0; m < SR; ++m)
            for (int fb = f0; fb < f1; fb += kPreThreads * kPreBatch) {
              unsigned xr[kPreBatch];
              load_x_raw(xr, P, m, fb, f1, pt);
              kick();
#pragma unroll
              for (int it = 0; it < kPreBatch; ++it) {
                const int f = fb + pt + kPreThreads * it;
                if (f < f1)
                  phl[m * lrow + unpack_pos<QT>((int)(w0 + f - P_lo))] = half_of(silu_f32(x_of_raw(xr[it], P.x_dtype)));
              }
            }
        }
      }
      kick();
      __syncthreads();  // every thread's basis values are in LDS before the sums read them
      // group sums as k_prep: each 8-block's fp16 values in order, then the
      // 8-block sums of a 64-group by xor steps 1, 2, 4 over its 8 lanes
      if constexpr (q_affine(QT)) {
#pragma unroll
        for (int m = 0; m < SR; ++m)
          for (int b0 = 0; b0 < nblk; b0 += kPreThreads) {
            const int blk = b0 + pt;
            const bool live = blk < nblk;
            uint4 u = make_uint4(0u, 0u, 0u, 0u);
            if (live) u = reinterpret_cast<const uint4*>(phl + m * lrow)[blk];
            const _Float16* hv = reinterpret_cast<const _Float16*>(&u);
            float sum = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += (float)hv[e];
            sum += __shfl_xor(sum, 1);
            sum += __shfl_xor(sum, 2);
            sum += __shfl_xor(sum, 4);
            const float other = __shfl_xor(sum, 8);
            if (live && (lane & 15) == 0) sl[(blk >> 4) * SR + m] = make_float2(sum, other);
          }
        __syncthreads();  // the group sums are in LDS before any wave reads them
      }
      if (!live_rg) return;  // a padding row group: its share of the basis is done
      static_for<0, RD - 1>([&](auto J) __attribute__((always_inline)) {
        issue_a(c_lo + decltype(J)::value, o[decltype(J)::value]);
      });
    } else {
      static_for<0, RD - 1>([&](auto J) __attribute__((always_inline)) {
        if constexpr (decltype(J)::value > 0) fence();
        issue(c_lo + decltype(J)::value, o[decltype(J)::value]);
      });
    }
    int c = c_lo;
    for (; c + RD <= c_hi; c += RD) {
      // slot j: refill the slot consumed last round with superchunk c + j + RD - 1, then multiply c + j
      static_for<0, RD>([&](auto J) __attribute__((always_inline)) {
        constexpr int j = decltype(J)::value;
        fence();
        issue(c + j + RD - 1, o[(j + RD - 1) % RD]);
        compute(o[j]);
      });
    }
    // slots 0 .. RD-2 hold superchunks c .. c + RD - 2
    static_for<0, RD - 1>([&](auto J) __attribute__((always_inline)) {
      if (c + decltype(J)::value < c_hi) compute(o[decltype(J)::value]);
    });
  }

  if (PRE && !live_rg) return;  // padding row group (an empty range skipped the basis work)
  // lane (q, r): row block q, column 16*(rb0 + q) + r, rows i < B from acc[q][i]
  const int n = (rb0 + q) * 16 + r;
  if (n < M.D_out) {
#pragma unroll
    for (int i = 0; i < SR; ++i) {
      float v = acc[0][i];
      v = q == 1 ? acc[1][i] : v;
      v = q == 2 ? acc[2][i] : v;
      v = q == 3 ? acc[3][i] : v;
      float* dst = part + ((long)ks * B + i) * N_total + M.col_off + n;
      if constexpr (EPI == QEPI_PART) *dst = v;
      else part_store(dst, v);
    }
  }
  if constexpr (EPI == QEPI_SWIGLU) {
    _Float16* stg;
    if constexpr (PRE) {
      // this wave's stage after the shared slice (other waves may still read the slice)
      stg = reinterpret_cast<_Float16*>(qg_dyn + P.slice + wave * kEpiStageBytes);
    } else {
      __shared__ _Float16 stage[4][64 * (kMaxK + 1)];
      stg = stage[threadIdx.x >> 6];
    }
    if (!last_arrival(E.counters + rg_loc * kCntStride, 2 * ksplit, lane)) return;
    epi_swiglu<QT, true>(E, part, ksplit, B, MP, m0.D_out, rg_loc, rg_split, stg, lane, 0, B);
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV for 2 < B <= 32 (k_qgemv_wg).  The four waves of a workgroup
// take four consecutive row groups over ONE superchunk range, so they share
// every superchunk's activation fragments (MT x 4 KB) and INT4 group sums:
// these are copied from L2 into a three-stage LDS ring by global_load_lds
// (no registers), one 1 KB instruction per fragment, in exactly the order the
// lanes read them (one conflict-free ds_read_b128 each).  The registers this
// frees hold a three-deep ring of the wave's own weight records (codes and
// group parameters), so two superchunks of weights stay in flight while one
// is multiplied.  Per superchunk: wait until this wave's loads of superchunk
// c have landed (vmcnt counts in issue order, so only the loads of c + 1 may
// still be pending), barrier (every wave's share of stage c is in LDS and
// every wave is done with stage c - 1), issue superchunk c + 2 into the
// freed stage, multiply.  A wave past the last row group streams the last
// row group again and stores nothing, so every wave issues the same loads
// and reaches the same barriers.  NT: non-temporal weight loads (load_rec).
// ---------------------------------------------------------------------------
template <int QT, int MT, bool NT>
__global__ void __launch_bounds__(256) k_qgemv_wg(QMatDev m0, QMatDev m1, int rg_split, int n_rg, int ksplit,
                                                  int C_tot, const _Float16* __restrict__ Phi,
                                                  const float2* __restrict__ S, int B, int MP,
                                                  float* __restrict__ part, int N_total) {
  constexpr int NW = kQNW;
  constexpr int FR = MT * 4;                    // activation fragments (1 KB each) per superchunk
  // vector-memory instructions per wave and superchunk: code words (one or two
  // 16-byte loads), fragment copies, group sums, the group-parameter copy
  // PR: group parameters through LDS (below); INT4 keeps them in the register
  // ring (through LDS its MT = 2 kernel took 256 registers, one wave per SIMD)
  constexpr bool PR = QT != Q_INT4;
  constexpr int OPS = qcode_loads(QT) + FR / 4 + (q_affine(QT) ? 1 : 0) + (PR ? 1 : NW);
  // three separate arrays per ring (not one indexed array): the compiler then
  // sees that reads of one stage do not depend on the copies into another,
  // and waits only for this stage's copies
  // PR: each wave's group parameters (its records' 1 KB parameter block) take
  // the same route, so the register ring holds only code words (ternary MT = 2:
  // 174 -> 150 registers, three waves per SIMD instead of two).  They sit in
  // the same stage array as the activation fragments, after them: with a
  // separate parameter array per stage the compiler could not tell the
  // parameter reads of stage c from the copies in flight into stage c + 1, and
  // made their first use wait for those copies (ternary: a vmcnt wait in the
  // middle of every superchunk's multiply, which drained the ring).
  constexpr int SPO = FR * 64;  // uint4 offset of the parameter blocks in a stage
  __shared__ uint4 sa0[SPO + (PR ? 4 * 64 : 0)], sa1[SPO + (PR ? 4 * 64 : 0)], sa2[SPO + (PR ? 4 * 64 : 0)];
  __shared__ float2 ss0[32], ss1[32], ss2[32];
  float4* const sp0 = reinterpret_cast<float4*>(sa0 + SPO);
  float4* const sp1 = reinterpret_cast<float4*>(sa1 + SPO);
  float4* const sp2 = reinterpret_cast<float4*>(sa2 + SPO);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ks = blockIdx.x % ksplit;
  const int rg_want = (blockIdx.x / ksplit) * 4 + wave;
  const bool live = rg_want < n_rg;
  const int rg = live ? rg_want : n_rg - 1;
  const QMatDev& M = rg < rg_split ? m0 : m1;
  const int rg_loc = rg < rg_split ? rg : rg - rg_split;
  const int rb0 = rg_loc * NW;
  const int c_lo = (int)((long)C_tot * ks / ksplit);
  const int c_hi = (int)((long)C_tot * (ks + 1) / ksplit);
  if (c_lo >= c_hi) return;  // uniform per workgroup
  const int q = lane >> 4, r = lane & 15;
  const long ldphi = (long)C_tot * 128;
  UnpackConsts uk;
  uk.init();

  typedef QWordOf<QT> QWord;
  const char* rbase = M.rec + (long)rg_loc * C_tot * qrec_bytes(QT);
  struct Wts {
    QWord qw[NW];
    float4 sb[NW];  // !PR only
  };
  auto load_w = [&](int c, Wts& o) {
    const char* rec = rbase + (long)c * qrec_bytes(QT);
    load_codes<NT, QT>(rec, lane, o.qw);
    if constexpr (!PR)
#pragma unroll
      for (int w = 0; w < NW; ++w) o.sb[w] = load_rec<NT, float4>(rec + NW * qtile_bytes(QT) + (w * 16 + r) * 16);
  };
  // the record's parameter block (kQNW x 16 rows x float4, 1 KB) into this
  // wave's slot of a stage: lane l copies bytes 16 l .. 16 l + 15
  auto dma_params = [&](int c, float4* sp) {
    const char* src = rbase + (long)c * qrec_bytes(QT) + NW * qtile_bytes(QT) + lane * 16;
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)&sp[wave * 64], 16, 0,
                                     NT ? 2 : 0);  // aux 2: non-temporal
  };
  // fragment j = 4 mt + t of superchunk c: lane l holds row 16 mt + l % 16,
  // reduction indices 128 c + 32 t + 8 (l / 16) .. + 7; wave w copies the
  // fragments j = w, w + 4, ...; every wave copies the INT4 group sums
  // (identical data, so each wave issues the same number of loads).
  auto dma = [&](int c, uint4* sa, float2* ss) {
#pragma unroll
    for (int jj = 0; jj < FR / 4; ++jj) {  // a constant count: the compiler's wait counts stay exact
      const int j = wave + 4 * jj;
      const int row = (j >> 2) * 16 + r;
      const _Float16* src = Phi + (long)row * ldphi + (long)c * 128 + 32 * (j & 3) + 8 * q;
      __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)&sa[j * 64], 16, 0, 0);
    }
    if constexpr (q_affine(QT)) {
      const float* ssrc = reinterpret_cast<const float*>(S + (long)c * MP) + min(lane, 2 * MP - 1);
      __builtin_amdgcn_global_load_lds(ssrc, (__attribute__((address_space(3))) void*)ss, 4, 0, 0);
    }
  };
  auto issue = [&](int c, uint4* sa, float2* ss, float4* sp, Wts& o) {
    const int cc = min(c, c_hi - 1);
    load_w(cc, o);
    dma(cc, sa, ss);
    if constexpr (PR) dma_params(cc, sp);
  };
  // waits for everything but the OPS loads of the superchunk after this one,
  // then the workgroup barrier; no fence (that would wait for all loads)
  auto sync_stage = [&]() {
    constexpr int kWait = (OPS & 15) | (0x7 << 4) | (0xf << 8) | ((OPS >> 4) << 14);
    __builtin_amdgcn_s_waitcnt(kWait);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // Passes a ring slot's registers through an empty asm after the wait that
  // covers them, so their first use (the unpack) cannot be hoisted above it:
  // hoisted, the code words are read while later loads are still in flight
  // and the compiler's own wait for them becomes vmcnt(0), which drains the
  // whole ring.
  auto pin = [&](Wts& o) {
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      unsigned* d = reinterpret_cast<unsigned*>(&o.qw[w]);
#pragma unroll
      for (int i = 0; i < (int)(sizeof(QWord) / 4); ++i) asm volatile("" : "+v"(d[i]));
      if constexpr (!PR) {
        float* sv = reinterpret_cast<float*>(&o.sb[w]);
#pragma unroll
        for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(sv[i]));
      }
    }
  };

  floatx4 acc[MT][NW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int w = 0; w < NW; ++w) acc[mt][w] = floatx4{0.f, 0.f, 0.f, 0.f};

  // one stage's fragments and group sums, read before the next DMA is issued
  // (the compiler cannot tell the stages apart and would otherwise wait for
  // that DMA before these reads)
  struct Frags {
    half8v a[MT][4];
    float2 sg[MT][4];  // INT4 / INT8: group sums of rows 16 mt + 4 q + i
    float4 sb[NW];     // PR: group parameters of row r of tile w
  };
  auto read_frags = [&](const uint4* sa, const float2* ss, const float4* sp, Frags& f) {
    if constexpr (PR) {
#pragma unroll
      for (int w = 0; w < NW; ++w) f.sb[w] = sp[wave * 64 + w * 16 + r];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint4 u = sa[(mt * 4 + t) * 64 + lane];
        f.a[mt][t] = *reinterpret_cast<const half8v*>(&u);
      }
    if constexpr (q_affine(QT)) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) f.sg[mt][i] = ss[mt * 16 + 4 * q + i];
    }
  };
  auto compute = [&](const Wts& ow, const Frags& f) {
    const auto& a = f.a;
    if constexpr (q_affine(QT)) {
      static_for<0, 2>([&](auto GS) __attribute__((always_inline)) {
        constexpr int gs = decltype(GS)::value;
        floatx4 g[MT][NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const half8v b0 = unpack_step<QT, 2 * gs>(ow.qw[w], uk);
          const half8v b1 = unpack_step<QT, 2 * gs + 1>(ow.qw[w], uk);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            g[mt][w] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][2 * gs], b0, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            g[mt][w] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][2 * gs + 1], b1, g[mt][w], 0, 0, 0);
          }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float S_ = gs ? f.sg[mt][i].y : f.sg[mt][i].x;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
              const float4& sbw = PR ? f.sb[w] : ow.sb[w];
              const float s = gs ? sbw.z : sbw.x;
              const float s2 = gs ? sbw.w : sbw.y;
              acc[mt][w][i] = __builtin_fmaf(s, g[mt][w][i], __builtin_fmaf(s2, S_, acc[mt][w][i]));
            }
          }
      });
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        floatx4 g[MT][NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const unsigned* dw = reinterpret_cast<const unsigned*>(&ow.qw[w]);
          const half8v bf = (t & 1) ? unpack_tern<1>(dw[t >> 1], uk) : unpack_tern<0>(dw[t >> 1], uk);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            g[mt][w] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][t], bf, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float4& sbw = PR ? f.sb[w] : ow.sb[w];
          const float s = t == 0 ? sbw.x : t == 1 ? sbw.y : t == 2 ? sbw.z : sbw.w;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mt][w][i] = __builtin_fmaf(s, g[mt][w][i], acc[mt][w][i]);
        }
      }
    }
  };

  Wts w0, w1, w2;
  Frags f;
  issue(c_lo, sa0, ss0, sp0, w0);
  // every load of superchunk c_lo before any of c_lo + 1: the waits count
  // loads in issue order
  __builtin_amdgcn_sched_barrier(0);
  issue(c_lo + 1, sa1, ss1, sp1, w1);
  // whole rounds of three superchunks: a branch-free body keeps the
  // compiler's own wait counts exact (a break inside it made them vmcnt(0))
  int c = c_lo;
  for (; c + 3 <= c_hi; c += 3) {
    sync_stage();
    pin(w0);
    read_frags(sa0, ss0, sp0, f);
    issue(c + 2, sa2, ss2, sp2, w2);
    compute(w0, f);
    sync_stage();
    pin(w1);
    read_frags(sa1, ss1, sp1, f);
    issue(c + 3, sa0, ss0, sp0, w0);
    compute(w1, f);
    sync_stage();
    pin(w2);
    read_frags(sa2, ss2, sp2, f);
    issue(c + 4, sa1, ss1, sp1, w1);
    compute(w2, f);
  }
  // the last one or two superchunks (stages 0 and 1, issued above)
  if (c < c_hi) {
    sync_stage();
    read_frags(sa0, ss0, sp0, f);
    compute(w0, f);
    if (c + 1 < c_hi) {
      __builtin_amdgcn_s_waitcnt(kWaitVmem);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      read_frags(sa1, ss1, sp1, f);
      compute(w1, f);
    }
  }
  // every load of the ring has landed before the workgroup's LDS is released
  __builtin_amdgcn_s_waitcnt(kWaitVmem);

  if (!live) return;
  // acc[mt][w][i] -> row m = 16mt + 4q + i, column 16*(rb0 + w) + r of matrix M
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int n = (rb0 + w) * 16 + r;
    if (n < M.D_out) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int mm = mt * 16 + 4 * q + i;
          if (mm < B) part[((long)ks * B + mm) * N_total + M.col_off + n] = acc[mt][w][i];
        }
    }
  }
}

// SwiGLU of the gate|up partial sums and the down layer's activation basis
// (Phi / S), one single-wave workgroup per (64-feature group, batch row): the
// small-batch GEMV's fused epilogue as a kernel of its own for B > 2, in place
// of k_qswiglu + k_prep (identical results, one launch and no hidden buffer).
template <int QT>
__global__ void __launch_bounds__(64) k_swiglu_basis(QEpi E, const float* __restrict__ part, int ksplit, int B,
                                                    int MP, int h, int n_groups) {
  __shared__ _Float16 stage[64 * (kMaxK + 1)];
  const int j = blockIdx.x, m = blockIdx.y;
  epi_swiglu<QT, false>(E, part, ksplit, B, MP, h, j, n_groups, stage, threadIdx.x, m, m + 1);
}

// y[m][col] = sum_ks part[ks][m][col] + bias.  Block = 64 columns x 4 split
// lanes: lane g sums the splits ks = g, g+4, ... in order, then the four
// partial sums are added in order (deterministic).
template <typename TY>
__global__ void __launch_bounds__(256) k_qreduce(const float* __restrict__ part, int ksplit, int B, int N,
                                                 const void* bias, int bias_dtype, TY* __restrict__ Y, long ldy) {
  __shared__ float red[4][64];
  const int col = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int m = blockIdx.y;
  const int n = blockIdx.x * 64 + col;
  const long total = (long)B * N;
  float sum = 0.0f;
  if (n < N) {
    // splits g, g+4, ... in order, loaded 16 at a time (one memory round trip
    // each; the B = 32 down GEMV has ~40 splits, 10 per thread)
    const float* p = part + (long)m * N + n;
    for (int k0 = g; k0 < ksplit; k0 += 64) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = k0 + 4 * u < ksplit ? p[(long)(k0 + 4 * u) * total] : 0.f;
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (k0 + 4 * u < ksplit) sum += v[u];
    }
  }
  red[g][col] = sum;
  __syncthreads();
  if (g == 0 && n < N) {
    float t = bias ? load_any(bias, n, bias_dtype) : 0.0f;
    t += red[0][col];
    t += red[1][col];
    t += red[2][col];
    t += red[3][col];
    Y[(long)m * ldy + n] = from_f32<TY>(t);
  }
}

// GatedKAN hidden state from the gate / up partial sums (columns [0, h) and
// [h, 2h) of part[ks][m][.]): hidden = SiLU(gate) * up (gated_kan.py:86-138,
// swiglu_forward_f32 fused_kan.metal:2284-2296, with the +-20 clip).  With
// round16 the gate and up layer outputs and the hidden state are rounded to
// fp16 (1) / bf16 (2), as the layer dtype does in the unfused path.
__global__ void k_qswiglu(const float* __restrict__ part, int ksplit, int B, int h, const void* bias_g,
                          const void* bias_u, int bias_g_dtype, int bias_u_dtype, int round16,
                          float* __restrict__ hidden) {
  const long total = (long)B * h;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    const int m = (int)(idx / h), i = (int)(idx - (long)m * h);
    float g = bias_g ? load_any(bias_g, i, bias_g_dtype) : 0.0f;
    float u = bias_u ? load_any(bias_u, i, bias_u_dtype) : 0.0f;
    const float* p = part + (long)m * 2 * h + i;
    for (int k0 = 0; k0 < ksplit; k0 += 8) {
      float vg[8], vu[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        vg[q] = k0 + q < ksplit ? p[(long)(k0 + q) * B * 2 * h] : 0.f;
        vu[q] = k0 + q < ksplit ? p[(long)(k0 + q) * B * 2 * h + h] : 0.f;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (k0 + q < ksplit) {
          g += vg[q];
          u += vu[q];
        }
    }
    if (round16) {
      g = round16_of(g, round16);
      u = round16_of(u, round16);
    }
    float hv = silu_clip(g) * u;
    if (round16) hv = round16_of(hv, round16);
    hidden[idx] = hv;
  }
}

// ---------------------------------------------------------------------------
// Host-side launchers.
// ---------------------------------------------------------------------------
static int grid_for(long n) { return (int)std::min<long>((n + 255) / 256, 8192); }

hipError_t qtile_int4(const unsigned char* qw, const float* scales, const float* biases, int D_out, long rowbytes,
                      int gpr, int nrb, int C, int c_off, int C_tot, void* R, hipStream_t st) {
  hipLaunchKernelGGL(k_tile_int4, dim3(grid_for((long)nrb * C * 64)), dim3(256), 0, st, qw, rowbytes, D_out, nrb, C,
                     c_off, C_tot, (char*)R);
  hipLaunchKernelGGL(k_tile_affine_params<Q_INT4>, dim3(grid_for((long)nrb * C * 16)), dim3(256), 0, st, scales,
                     biases, gpr, D_out, nrb, C, c_off, C_tot, (char*)R);
  return hipGetLastError();
}

hipError_t qtile_int8(const unsigned char* qw, const float* scales, const float* biases, int D_out, long rowbytes,
                      int gpr, int nrb, int C, int c_off, int C_tot, void* R, hipStream_t st) {
  hipLaunchKernelGGL(k_tile_int8, dim3(grid_for((long)nrb * C * 64)), dim3(256), 0, st, qw, rowbytes, D_out, nrb, C,
                     c_off, C_tot, (char*)R);
  hipLaunchKernelGGL(k_tile_affine_params<Q_INT8>, dim3(grid_for((long)nrb * C * 16)), dim3(256), 0, st, scales,
                     biases, gpr, D_out, nrb, C, c_off, C_tot, (char*)R);
  return hipGetLastError();
}

hipError_t qtile_tern(const unsigned* wp, const float* scales, int D_out, int wpr, long K_dim, int gpr, int nrb,
                      int C, int c_off, int C_tot, void* R, hipStream_t st) {
  hipLaunchKernelGGL(k_tile_tern, dim3(grid_for((long)nrb * C * 64)), dim3(256), 0, st, wp, wpr, K_dim, D_out, nrb,
                     C, c_off, C_tot, (char*)R);
  hipLaunchKernelGGL(k_tile_tern_params, dim3(grid_for((long)nrb * C * 16)), dim3(256), 0, st, scales, gpr, D_out,
                     nrb, C, c_off, C_tot, (char*)R);
  return hipGetLastError();
}

hipError_t qprep(int qt, const QPrep& P, hipStream_t st) {
  // rows B .. MP-1 are left as they are: the GEMVs read them only into
  // accumulator rows they never store
  dim3 grid((unsigned)((P.C_tot * 16 + 255) / 256), (unsigned)P.B);
  PrepIn in{P.X, P.x_dtype, P.ldx, P.basis, P.bp};
  if (qt == Q_INT4)
    hipLaunchKernelGGL((k_prep<Q_INT4>), grid, dim3(256), 0, st, in, P.B, P.MP, P.D_in, P.K, P.has_base, P.Cb,
                       P.C_tot, P.Phi, P.S);
  else if (qt == Q_INT8)
    hipLaunchKernelGGL((k_prep<Q_INT8>), grid, dim3(256), 0, st, in, P.B, P.MP, P.D_in, P.K, P.has_base, P.Cb,
                       P.C_tot, P.Phi, P.S);
  else
    hipLaunchKernelGGL((k_prep<Q_TERN>), grid, dim3(256), 0, st, in, P.B, P.MP, P.D_in, P.K, P.has_base, P.Cb,
                       P.C_tot, P.Phi, P.S);
  return hipGetLastError();
}

// Bytes of a workgroup's LDS slice for the in-kernel basis (QPreDev): the
// basis values and group sums of its superchunk range.
static int pre_slice_bytes(int qt, int B, int span) {
  const int b = span * B * 256 + (q_affine(qt) ? span * B * 8 : 0);
  return (b + 15) & ~15;
}
// Dynamic LDS of a k_qgemv<PRE> workgroup: the slice, then one epilogue stage
// per wave (QEPI_SWIGLU).
static int pre_lds_bytes(int qt, int B, int span, int epi_kind) {
  return pre_slice_bytes(qt, B, span) + (epi_kind == QEPI_SWIGLU ? 4 * kEpiStageBytes : 0);
}

bool qgemv_pre_fits(int qt, int B, int C_tot, int ksplit, int epi_kind) {
  static int lds_max = -1;  // per-workgroup LDS limit of the device
  if (lds_max < 0) {
    int dev = 0, v = 0;
    lds_max = hipGetDevice(&dev) == hipSuccess &&
                      hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess
                  ? v
                  : 0;
  }
  if (B < 1 || B > kSmallB || ksplit < 1) return false;
  const int span = (C_tot + ksplit - 1) / ksplit;
  return pre_lds_bytes(qt, B, span, epi_kind) <= std::min(kPreLdsMax, lds_max);
}

// Launch of the decode GEMV kernel for G (arguments checked by qgemv).
template <bool NT>
static void qgemv_launch(int qt, const QGemv& G, hipStream_t st) {
  QMatDev a{(const char*)G.rec0, G.D_out0, 0};
  QMatDev b{(const char*)(G.rec1 ? G.rec1 : G.rec0), G.D_out1, G.D_out0};
  const int items = G.n_rg * G.ksplit;
  QPreDev P{G.X, G.x_dtype, G.ldx, G.D_in, G.K, G.has_base, G.Cb, 0, 0};
  const bool pre = G.X != nullptr;
  if (pre) {
    P.span = (G.C_tot + G.ksplit - 1) / G.ksplit;
    P.slice = pre_slice_bytes(qt, G.B, P.span);
  }
  // PRE: a workgroup per (four row groups, split); otherwise per four items
  dim3 grid((unsigned)(pre ? (G.n_rg + 3) / 4 * G.ksplit : (items + 3) / 4));
  const size_t dyn = pre ? (size_t)pre_lds_bytes(qt, G.B, P.span, G.epi.kind) : 0;
#define KQ_GEMV(QTV, SR, EP)                                                                                      \
  do {                                                                                                           \
    if (pre)                                                                                                     \
      hipLaunchKernelGGL((k_qgemv<QTV, SR, EP, NT, true>), grid, dim3(256), dyn, st, a, b, G.rg_split, G.n_rg,    \
                         G.ksplit, G.C_tot, G.Phi, G.S, G.B, G.MP, G.part, G.N_total, G.epi, P);                 \
    else                                                                                                         \
      hipLaunchKernelGGL((k_qgemv<QTV, SR, EP, NT, false>), grid, dim3(256), 0, st, a, b, G.rg_split, G.n_rg,     \
                         G.ksplit, G.C_tot, G.Phi, G.S, G.B, G.MP, G.part, G.N_total, G.epi, P);                 \
  } while (0)
  const int mt = G.MP / 16;
  const bool small = G.B <= kSmallB;
  const int ep = G.epi.kind;
  // small batches: one kernel per row count (B = 1, 2), each with and without
  // the fused SwiGLU epilogue
#define KQ_SMALL(QTV)                                                                                 \
  do {                                                                                                \
    if (G.B == 1) {                                                                                   \
      if (ep == QEPI_SWIGLU) KQ_GEMV(QTV, 1, QEPI_SWIGLU); else KQ_GEMV(QTV, 1, QEPI_PART);            \
    } else {                                                                                          \
      if (ep == QEPI_SWIGLU) KQ_GEMV(QTV, 2, QEPI_SWIGLU); else KQ_GEMV(QTV, 2, QEPI_PART);            \
    }                                                                                                 \
  } while (0)
  // larger batches: workgroups of four row groups sharing one superchunk range
  const dim3 grid_wg((unsigned)((G.n_rg + 3) / 4 * G.ksplit));
#define KQ_WG(QTV, MTV)                                                                                        \
  hipLaunchKernelGGL((k_qgemv_wg<QTV, MTV, NT>), grid_wg, dim3(256), 0, st, a, b, G.rg_split, G.n_rg, G.ksplit,    \
                     G.C_tot, G.Phi, G.S, G.B, G.MP, G.part, G.N_total)
  if (qt == Q_INT4) {
    if (small) KQ_SMALL(Q_INT4);
    else if (mt == 1) KQ_WG(Q_INT4, 1);
    else KQ_WG(Q_INT4, 2);
  } else if (qt == Q_INT8) {
    if (small) KQ_SMALL(Q_INT8);
    else if (mt == 1) KQ_WG(Q_INT8, 1);
    else KQ_WG(Q_INT8, 2);
  } else {
    if (small) KQ_SMALL(Q_TERN);
    else if (mt == 1) KQ_WG(Q_TERN, 1);
    else KQ_WG(Q_TERN, 2);
  }
#undef KQ_WG
#undef KQ_SMALL
#undef KQ_GEMV
}

hipError_t qgemv(int qt, const QGemv& G, hipStream_t st) {
  const bool small = G.B <= kSmallB;
  // k_qgemv addresses a row group's records with 32-bit buffer offsets
  if (small && (long)G.C_tot * qrec_bytes(qt) > 0x7fffffffL) return hipErrorInvalidValue;
  const int ep = G.epi.kind;
  if (ep != QEPI_PART && (!small || !G.epi.counters || G.ksplit > kMaxEpiSplit || !G.rec1 || G.D_out1 != G.D_out0))
    return hipErrorInvalidValue;
  if (G.X && (!qgemv_pre_fits(qt, G.B, G.C_tot, G.ksplit, ep) || G.K < 1 || G.D_in < 1 || G.ldx < G.D_in))
    return hipErrorInvalidValue;
  if (!small && G.MP > 32) return hipErrorInvalidValue;
  if (G.nt) qgemv_launch<true>(qt, G, st);
  else qgemv_launch<false>(qt, G, st);
  return hipGetLastError();
}

hipError_t qswiglu_basis(int qt, const QEpi& E, const float* part, int ksplit, int B, int MP, int h,
                         hipStream_t st) {
  if (E.K2 < 1 || E.K2 > kMaxK || B < 1 || B > MP || !E.Phi2 || (q_affine(qt) && !E.S2)) return hipErrorInvalidValue;
  const int n_groups = (h + 63) / 64;
  const dim3 grid((unsigned)n_groups, (unsigned)B);
  if (qt == Q_INT4)
    hipLaunchKernelGGL(k_swiglu_basis<Q_INT4>, grid, dim3(64), 0, st, E, part, ksplit, B, MP, h, n_groups);
  else if (qt == Q_INT8)
    hipLaunchKernelGGL(k_swiglu_basis<Q_INT8>, grid, dim3(64), 0, st, E, part, ksplit, B, MP, h, n_groups);
  else
    hipLaunchKernelGGL(k_swiglu_basis<Q_TERN>, grid, dim3(64), 0, st, E, part, ksplit, B, MP, h, n_groups);
  return hipGetLastError();
}

hipError_t qreduce(const float* part, int ksplit, int B, int N, const void* bias, int bias_dtype, void* Y, int y_dtype,
                   long ldy, hipStream_t st) {
  const dim3 blocks((unsigned)((N + 63) / 64), (unsigned)B);
  if (y_dtype == DT_F16)
    hipLaunchKernelGGL((k_qreduce<_Float16>), blocks, dim3(256), 0, st, part, ksplit, B, N, bias, bias_dtype,
                       (_Float16*)Y, ldy);
  else if (y_dtype == DT_BF16)
    hipLaunchKernelGGL((k_qreduce<__bf16>), blocks, dim3(256), 0, st, part, ksplit, B, N, bias, bias_dtype,
                       (__bf16*)Y, ldy);
  else
    hipLaunchKernelGGL((k_qreduce<float>), blocks, dim3(256), 0, st, part, ksplit, B, N, bias, bias_dtype, (float*)Y,
                       ldy);
  return hipGetLastError();
}

hipError_t qswiglu(const float* part, int ksplit, int B, int h, const void* bias_g, int bias_g_dtype,
                   const void* bias_u, int bias_u_dtype, int round16, float* hidden, hipStream_t st) {
  hipLaunchKernelGGL(k_qswiglu, dim3(grid_for((long)B * h)), dim3(256), 0, st, part, ksplit, B, h, bias_g, bias_u,
                     bias_g_dtype, bias_u_dtype, round16, hidden);
  return hipGetLastError();
}

}  // namespace kans
