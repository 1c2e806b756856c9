// Quantized prefill: the split reduction, the re-tiling kernels that build the
// prefill layout from the reference formats, and the host launch.  The fused
// kernel itself is kans_qprefill_kernel.h, instantiated per weight format and
// base flag in kans_qprefill_{int4,int8,tern}_b{0,1}.hip.
#include "kans_qprefill_kernel.h"

namespace kans {

// Split reduction: the partial sums of the column-interleaved N-tiles
// (part[split][B][n_tiles * 256]) -> y (plain) or hidden (SwiGLU of the
// gate / up column pairs), splits added in order.
__global__ void k_qp_finalize(const float* __restrict__ part, int splits, int B, int n_tiles, int epi, int grp,
                              const void* bias0, const void* bias1, int bias_dt, int D_out, void* Y, long ldy,
                              int y_dt, int round16) {
  const long ncols = (long)n_tiles * 256;
  const long n = (long)B * D_out;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (long)gridDim.x * blockDim.x) {
    const int row = (int)(idx / D_out), c = (int)(idx - (long)row * D_out);
    // column of output c in the interleaved layout
    const long pc = grp == 4 ? ((long)(c >> 7) * 256 + (c & 127)) : c;
    const float* p = part + (long)row * ncols + pc;
    const long sstride = (long)B * ncols;
    float g = bias0 ? load_any_f(bias0, c, bias_dt) : 0.0f;
    float u = (epi == QP_EPI_SWIGLU && bias1) ? load_any_f(bias1, c, bias_dt) : 0.0f;
    for (int k = 0; k < splits; ++k) {
      g += p[k * sstride];
      if (epi == QP_EPI_SWIGLU) u += p[k * sstride + 128];
    }
    if (epi == QP_EPI_SWIGLU) {
      g = round16v(g, round16);
      u = round16v(u, round16);
      g = round16v(silu_clip20(g) * u, round16);
    }
    store_any(Y, (long)row * ldy + c, y_dt, g);
  }
}

// ---------------------------------------------------------------------------
// Re-tiling kernels (one thread per 8-code chunk / per parameter).
// ---------------------------------------------------------------------------
template <int BITS>
__global__ void k_qp_tile_affine(const unsigned char* __restrict__ qw, long rowbytes, int D_out, int D_in, int Kseg,
                                 int nfb, int nob_pad, unsigned char* __restrict__ codes) {
  const long total = (long)nfb * nob_pad * 64 * Kseg;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    // idx = ((fb * nob_pad + ob) * Kseg + s) * 64 + lane
    const int lane = (int)(idx % 64);
    long r = idx / 64;
    const int s = (int)(r % Kseg);
    r /= Kseg;
    const int ob = (int)(r % nob_pad);
    const int fb = (int)(r / nob_pad);
    const int o = ob * 32 + (lane & 31);
    const int i0 = fb * 16 + 8 * (lane >> 5);
    unsigned q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      q[e] = 0u;
      const int i = i0 + e;
      if (o < D_out && i < D_in) {
        const long j = (long)i * Kseg + s;
        if (BITS == 8) q[e] = qw[(long)o * rowbytes + j];
        else {
          const unsigned b = qw[(long)o * rowbytes + (j >> 1)];
          q[e] = (j & 1) ? (b >> 4) : (b & 15u);
        }
      }
    }
    if (BITS == 8) {
      const unsigned w0 = q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24);
      const unsigned w1 = q[4] | (q[5] << 8) | (q[6] << 16) | (q[7] << 24);
      reinterpret_cast<uint2*>(codes)[idx] = make_uint2(w0, w1);
    } else {
      unsigned w = 0u;
#pragma unroll
      for (int e = 0; e < 8; ++e) w |= q[e] << int4_pos(e);
      reinterpret_cast<unsigned*>(codes)[idx] = w;
    }
  }
}

template <int PF>
__global__ void k_qp_tile_params(const float* __restrict__ scales, const float* __restrict__ biases, int gpr,
                                 int D_out, int G_alloc, long ldp, float* __restrict__ params) {
  const long total = (long)G_alloc * ldp;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    const int g = (int)(idx / ldp), o = (int)(idx - (long)g * ldp);
    const bool ok = o < D_out && g < gpr;
    params[idx * PF] = ok ? scales[(long)o * gpr + g] : 0.0f;
    if (PF == 2) params[idx * PF + 1] = ok ? biases[(long)o * gpr + g] : 0.0f;
  }
}

__global__ void k_qp_tile_tern(const unsigned* __restrict__ wp, int wpr, int D_out, int D_in, int Kseg, int nfb,
                               int nob_pad, unsigned char* __restrict__ codes) {
  // one thread per (fb, ob, slot pair, lane) for Kseg > 1 (an odd Kseg padded
  // with a slot of zero weights), per (fb, ob, lane) for Kseg = 1
  const int per = Kseg == 1 ? 1 : (Kseg + 1) / 2;
  const long total = (long)nfb * nob_pad * 64 * per;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    // idx = ((fb * nob_pad + ob) * per + t) * 64 + lane
    const int lane = (int)(idx % 64);
    long r = idx / 64;
    const int t = (int)(r % per);
    r /= per;
    const int ob = (int)(r % nob_pad);
    const int fb = (int)(r / nob_pad);
    const int o = ob * 32 + (lane & 31);
    const int i0 = fb * 16 + 8 * (lane >> 5);
    auto code = [&](int e, int s) -> unsigned {
      const int i = i0 + e;
      if (o >= D_out || i >= D_in || s >= Kseg) return 1u;  // zero weight
      const long j = (long)i * Kseg + s;
      return (wp[(long)o * wpr + (j >> 4)] >> (2 * (j & 15))) & 3u;
    };
    if (Kseg == 1) {
      unsigned h = 0u;
#pragma unroll
      for (int p = 0; p < 4; ++p) h |= (code(2 * p, 0) << (2 * p)) | (code(2 * p + 1, 0) << (8 + 2 * p));
      reinterpret_cast<unsigned short*>(codes)[idx] = (unsigned short)h;
    } else {
      unsigned w = 0u;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        w |= code(2 * p, 2 * t) << (2 * p);                // slot 2t, layout A
        w |= code(2 * p + 1, 2 * t) << (16 + 2 * p);
        w |= code(2 * p, 2 * t + 1) << (8 + 2 * p);        // slot 2t + 1, layout B
        w |= code(2 * p + 1, 2 * t + 1) << (24 + 2 * p);
      }
      reinterpret_cast<unsigned*>(codes)[idx] = w;
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side launch.
// ---------------------------------------------------------------------------
static int grid_of(long n) { return (int)std::min<long>((n + 255) / 256, 8192); }

hipError_t qp_tile_affine(int bits, const unsigned char* qw, long rowbytes, const float* scales, const float* biases,
                          int gpr, int D_out, int D_in, int Kseg, int nfb, int nob_pad, int G_alloc, void* codes,
                          float* params, hipStream_t st) {
  const long nchunks = (long)nfb * nob_pad * 64 * Kseg;
  if (bits == 8)
    hipLaunchKernelGGL(k_qp_tile_affine<8>, dim3(grid_of(nchunks)), dim3(256), 0, st, qw, rowbytes, D_out, D_in,
                       Kseg, nfb, nob_pad, (unsigned char*)codes);
  else
    hipLaunchKernelGGL(k_qp_tile_affine<4>, dim3(grid_of(nchunks)), dim3(256), 0, st, qw, rowbytes, D_out, D_in,
                       Kseg, nfb, nob_pad, (unsigned char*)codes);
  const long ldp = (long)nob_pad * 32;
  hipLaunchKernelGGL(k_qp_tile_params<2>, dim3(grid_of((long)G_alloc * ldp)), dim3(256), 0, st, scales, biases, gpr,
                     D_out, G_alloc, ldp, params);
  return hipGetLastError();
}

hipError_t qp_tile_tern(const unsigned* wp, int wpr, const float* scales, int gpr, int D_out, int D_in, int Kseg,
                        int nfb, int nob_pad, int G_alloc, void* codes, float* params, hipStream_t st) {
  const long n = (long)nfb * nob_pad * 64 * (Kseg == 1 ? 1 : (Kseg + 1) / 2);
  hipLaunchKernelGGL(k_qp_tile_tern, dim3(grid_of(n)), dim3(256), 0, st, wp, wpr, D_out, D_in, Kseg, nfb, nob_pad,
                     (unsigned char*)codes);
  const long ldp = (long)nob_pad * 32;
  hipLaunchKernelGGL(k_qp_tile_params<1>, dim3(grid_of((long)G_alloc * ldp)), dim3(256), 0, st, scales, scales, gpr,
                     D_out, G_alloc, ldp, params);
  return hipGetLastError();
}

int qp_choose_splits(int B, int D_in, int n_cols, int grp) {
  const int m_tiles = (B + 255) / 256;
  const int n_tiles = (n_cols + 32 * grp - 1) / (32 * grp);
  const int tiles = m_tiles * n_tiles;
  const int nfb = (D_in + 15) / 16;
  if (tiles >= 256) return 1;
  // towards one workgroup per CU, at least 8 feature blocks per split
  return std::max(1, std::min((256 + tiles - 1) / tiles, nfb / 8));
}

long qp_part_floats(const QPLaunch& L) {
  if (L.splits <= 1) return 0;
  const int n_cols = L.m[0].D_out;
  const int n_tiles = (n_cols + 32 * L.grp - 1) / (32 * L.grp);
  return (long)L.splits * L.B * n_tiles * 256;
}

int g_qp_block_pairs = 1;

hipError_t qp_launch(const QPLaunch& L, hipStream_t st) {
  if (!qp_supported(L.qt, L.K, L.has_base, L.basis, L.bp.rbf_rec) || (L.grp != 4 && L.grp != 8) || L.B <= 0 ||
      (L.basis != BASIS_CHEBY && (L.grp != 8 || L.bp.K != L.K)))
    return hipErrorInvalidValue;
  QPGrid G;
  G.m_tiles = (L.B + 255) / 256;
  G.n_tiles = (L.m[0].D_out + 32 * L.grp - 1) / (32 * L.grp);
  G.nfb = (L.D_in + 15) / 16;
  const int splits = std::max(1, std::min(L.splits, G.nfb));
  // splits start at a multiple of the kernel's phase period (qp_period)
  const int per = qp_period(L.K, qp_group(L.qt));
  G.fb_per_split = ((G.nfb + splits - 1) / splits + per - 1) / per * per;
  G.nsp = (G.nfb + G.fb_per_split - 1) / G.fb_per_split;
  hipError_t e;
  switch (L.qt) {
    case Q_INT4: e = L.has_base ? qp_run_int4_b1(L, G, st) : qp_run_int4_b0(L, G, st); break;
    case Q_INT8: e = L.has_base ? qp_run_int8_b1(L, G, st) : qp_run_int8_b0(L, G, st); break;
    default: e = L.has_base ? qp_run_tern_b1(L, G, st) : qp_run_tern_b0(L, G, st); break;
  }
  if (e != hipSuccess || G.nsp <= 1) return e;
  const long n = (long)L.B * L.m[0].D_out;
  hipLaunchKernelGGL(k_qp_finalize, dim3(grid_of(n)), dim3(256), 0, st, (const float*)L.part, G.nsp, L.B, G.n_tiles,
                     L.epi, L.grp, L.m[0].bias, L.grp == 4 ? L.m[1].bias : nullptr, L.bias_dtype, L.m[0].D_out, L.Y,
                     L.ldy, L.y_dtype, L.round16);
  return hipGetLastError();
}

}  // namespace kans
