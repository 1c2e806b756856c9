// Fused KAN layer forward for gfx950: basis expansion + output contraction in
// one kernel, so the expanded Phi tensor never exists in memory.
//
//   y[b,o] = bias[o] + sum_i SiLU(x[b,i]) W_base[o,i] + sum_{i,k} phi_k(x[b,i]) W[o,i*K+k]
//
// Replaces the reference's four-stage dispatch (eval_base_and_bias, MPS GEMM,
// eval_*_basis into a B*D_in*K scratch buffer, MPS GEMM) of
// metal_kan_bridge.mm:443-625,1069-1164,1890-2151.
//
// Work decomposition (one workgroup = 4 waves = 256 threads, two resident per CU):
//   * a wave owns WM rows (32 or 64) x NB*32 output columns; the 4 waves stack
//     along rows, so a workgroup tile is 4*WM x NB*32;
//   * the inner dimension is walked as steps (feature block fb of 16 inputs,
//     slot s): slot 0 is SiLU(x) when the layer has the base branch, the rest
//     are the K basis functions.  Each lane holds 8 inputs of each of its row
//     blocks, evaluates the slot's basis value for them in fp32 registers (the
//     Chebyshev / RBF / B-spline generators advance slot by slot), and packs
//     them straight into the MFMA A-fragment;
//   * the B-fragments come from LDS, filled from the pre-tiled weights (one
//     (fb, s) step of an N-tile is NB contiguous KB);
//   * fp16 / bf16 use v_mfma_f32_32x32x16_{f16,bf16}; fp32 uses
//     v_mfma_f32_32x32x2_f32 eight times per step.  Accumulation is fp32.
//   * an optional split over feature blocks writes fp32 partials that a finalize
//     kernel reduces (used when the output tile count alone cannot fill the GPU);
//     the 4-wave block kernel can also split a tile's feature blocks over KS
//     wave groups of one workgroup, reduced through LDS (no finalize kernel).
//
// Two kernels share this decomposition:
//   kan_fused_block  fp16/bf16: Chebyshev with K+base <= 10 (4 waves), RBF and
//                    B-spline with K+base <= 9 on the 256 x 256 tile (8 waves):
//                    one barrier per feature block, global->LDS DMA of the next
//                    block's weights, basis generation interleaved with the MFMAs;
//   kan_fused_dense  everything else (fp32, other tiles, larger K): one
//                    barrier per slot, register-staged weights.
#include "kans_common.h"
#include "kans_api_internal.h"
#include "kans_tile.h"
#include <algorithm>
#include <type_traits>

namespace kans {

constexpr int kStages = 3;
constexpr int kThreads = 256;

// T: weight / MFMA operand type; TX: input element type; TY: output element
// type (TX, TY in {T, float}: a 16-bit chain keeps fp32 activations between
// layers).
template <typename T, typename TX, typename TY, int BASIS, int WM, int NB>
__global__ void __launch_bounds__(kThreads, 2)
kan_fused_dense(const TX* __restrict__ X, long ldx,
                const uint4* __restrict__ Wt, int nob_pad,
                const T* __restrict__ bias,
                TY* __restrict__ Y, long ldy,
                float* __restrict__ Ypart,
                int B, int D_in, int D_out, int m_tiles, int n_tiles,
                int nfb_total, int fb_per_split, int has_base, BasisParams bp) {
  constexpr int RB = WM / 32;           // 32-row blocks per wave
  constexpr int NV = RB * 8;            // inputs held per lane
  constexpr int CPL = Chunks<T>::CPL;   // uint4 per lane per 32-col block
  constexpr int CPX = Chunks<TX>::CPL;  // uint4 per lane per row block of inputs
  constexpr int SU = NB * 64 * CPL;     // uint4 per pipeline stage
  constexpr int LPT = (SU + kThreads - 1) / kThreads;
  constexpr bool kHalf = sizeof(T) == 2;

  __shared__ uint4 lds[kStages][SU];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index as a scalar: the compiler cannot see that tid >> 6 is uniform
  // per wave, and would otherwise keep wave-derived loop counters and
  // addresses in vector registers
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles = m_tiles * n_tiles;
  const int lin = xcd_remap(blockIdx.x, tiles);
  const int n_tile = lin / m_tiles;
  const int m_tile = lin - n_tile * m_tiles;
  const int split = blockIdx.y;

  const int row0 = m_tile * (4 * WM) + wave * WM;
  const int ob0 = n_tile * NB;
  const int fb_begin = split * fb_per_split;
  const int fb_end = min(nfb_total, fb_begin + fb_per_split);
  const int K = bp.K;
  const int KP = K + has_base;
  const int nsteps = (fb_end - fb_begin) * KP;

  // ---- global -> LDS weight pipeline ------------------------------------
  // Step t covers (fb, slot) = (fb_begin + t / KP, t % KP); its tile for this
  // N-tile is SU contiguous uint4 of W'.  Stage ring of kStages; step t+2 is
  // fetched into registers at the top of step t and written to LDS at its
  // bottom, so the load latency hides behind step t's MFMAs (and the other
  // resident workgroup).
  const uint4* wbase = Wt + (long)ob0 * (64 * CPL) + tid;
  const long slot_stride = (long)nob_pad * (64 * CPL);
  // The staged chunks live in one vector value, not a uint4 array: an array of
  // more than one uint4 was left in private (scratch) memory by the compiler.
  typedef unsigned RegVec __attribute__((ext_vector_type(4 * LPT)));
  RegVec rg;
  auto gload = [&](int t) {
    const uint4* src = wbase + ((long)fb_begin * KP + t) * slot_stride;
#pragma unroll
    for (int q = 0; q < LPT; ++q)
      if (q * kThreads + tid < SU) {
        const uint4 u = src[q * kThreads];
        rg[4 * q + 0] = u.x;
        rg[4 * q + 1] = u.y;
        rg[4 * q + 2] = u.z;
        rg[4 * q + 3] = u.w;
      }
  };
  auto lstore = [&](int t) {
    uint4* dst = lds[t % kStages] + tid;
#pragma unroll
    for (int q = 0; q < LPT; ++q)
      if (q * kThreads + tid < SU) dst[q * kThreads] = make_uint4(rg[4 * q], rg[4 * q + 1], rg[4 * q + 2], rg[4 * q + 3]);
  };

  // ---- input rows ---------------------------------------------------------
  // lane holds x[row0 + rb*32 + lane%32][fb*16 + 8*(lane/32) + j], j = 0..7
  uint4 xr[RB][CPX];
  auto xload = [&](int fbx) {
    const int f0 = fbx * 16 + 8 * (lane >> 5);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = row0 + rb * 32 + (lane & 31);
      const bool ok = (row < B) && (f0 < D_in);
      const uint4* p = reinterpret_cast<const uint4*>(X + (long)row * ldx + f0);
#pragma unroll
      for (int c = 0; c < CPX; ++c) xr[rb][c] = ok ? p[c] : make_uint4(0, 0, 0, 0);
      if (ok && f0 + 8 > D_in) {
        // tail chunk: inputs at or beyond D_in read as 0 whatever the padding holds
#pragma unroll
        for (int c = 0; c < CPX; ++c) {
          unsigned w[4] = {xr[rb][c].x, xr[rb][c].y, xr[rb][c].z, xr[rb][c].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if constexpr (sizeof(TX) == 4) {
              if (f0 + c * 4 + q >= D_in) w[q] = 0u;
            } else {
              if (f0 + 2 * q >= D_in) w[q] &= 0xffff0000u;
              if (f0 + 2 * q + 1 >= D_in) w[q] &= 0x0000ffffu;
            }
          }
          xr[rb][c] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    }
  };

  floatx16 acc[RB][NB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[rb][nb][r] = 0.0f;

  if (nsteps <= 0) return;  // uniform per workgroup (empty split)

  // prologue: steps 0 and 1 into LDS.
  gload(0);
  lstore(0);
  if (nsteps > 1) { gload(1); lstore(1); }
  xload(fb_begin);
  __syncthreads();

  int t = 0;  // global step counter
  // One step: fetch step t+2, multiply the slot's A-fragment (basis values v)
  // by the B-fragments of step t, store step t+2, barrier.
  auto step = [&](const float* v) {
    const bool pf = t + 2 < nsteps;
    if (pf) gload(t + 2);
    const uint4* st = lds[t % kStages];
    if constexpr (kHalf) {
      typedef typename Mfma<T>::frag frag;
      frag a[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < 8; ++j) a[rb][j] = from_f32<T>(v[rb * 8 + j]);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        uint4 u = st[nb * 64 + lane];
        frag b = *reinterpret_cast<frag*>(&u);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb][nb] = Mfma<T>::mma(a[rb], b, acc[rb][nb]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float bv[NB][4];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          uint4 u = st[(nb * 2 + c) * 64 + lane];
          bv[nb][0] = __uint_as_float(u.x);
          bv[nb][1] = __uint_as_float(u.y);
          bv[nb][2] = __uint_as_float(u.z);
          bv[nb][3] = __uint_as_float(u.w);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              acc[rb][nb] = __builtin_amdgcn_mfma_f32_32x32x2f32(v[rb * 8 + c * 4 + e], bv[nb][e], acc[rb][nb],
                                                                  0, 0, 0);
      }
    }
    if (pf) lstore(t + 2);
    ++t;
    __syncthreads();
  };

  BasisGen<BASIS, NV> gen;
  for (int fb = fb_begin; fb < fb_end; ++fb) {
    float xf[NV];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int c = 0; c < CPX; ++c) {
        const uint4 u = xr[rb][c];
        if constexpr (sizeof(TX) == 4) {
          xf[rb * 8 + c * 4 + 0] = __uint_as_float(u.x);
          xf[rb * 8 + c * 4 + 1] = __uint_as_float(u.y);
          xf[rb * 8 + c * 4 + 2] = __uint_as_float(u.z);
          xf[rb * 8 + c * 4 + 3] = __uint_as_float(u.w);
        } else {
          const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            TX lo, hi;
            const unsigned short l16 = (unsigned short)(w[q] & 0xffffu), h16 = (unsigned short)(w[q] >> 16);
            __builtin_memcpy(&lo, &l16, 2);
            __builtin_memcpy(&hi, &h16, 2);
            xf[rb * 8 + 2 * q] = to_f32(lo);
            xf[rb * 8 + 2 * q + 1] = to_f32(hi);
          }
        }
      }
    if (fb + 1 < fb_end) xload(fb + 1);
    gen.begin(xf, bp);
    if (has_base) {
      float v[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) v[i] = silu_f32(xf[i]);
      step(v);
    }
    int k = 0;
    for (; k + 1 < K; k += 2) {
      float v0[NV], v1[NV];
      gen.pair(k, bp, v0, v1);
      step(v0);
      step(v1);
    }
    if (k < K) {
      float v0[NV];
      gen.one(k, bp, v0);
      step(v0);
    }
  }

  // ---- epilogue -------------------------------------------------------------
  // acc register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  const int rbase = row0 + 4 * (lane >> 5);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int col = (ob0 + nb) * 32 + (lane & 31);
    if (col < D_out) {
      if (Ypart != nullptr) {
        float* out = Ypart + ((long)split * B + rbase) * D_out + col;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dr = rb * 32 + 8 * (r >> 2) + (r & 3);
            if (rbase + dr < B) out[(long)dr * D_out] = acc[rb][nb][r];
          }
      } else {
        const float bcol = bias != nullptr ? to_f32(bias[col]) : 0.0f;
        TY* out = Y + (long)rbase * ldy + col;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dr = rb * 32 + 8 * (r >> 2) + (r & 3);
            if (rbase + dr < B) out[(long)dr * ldy] = from_f32<TY>(acc[rb][nb][r] + bcol);
          }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fp16 / bf16 kernel with one barrier per feature block.
//
// The weights of a whole feature block (KP slots x NB KB for the workgroup's
// N-tile) sit in one of two LDS stages.  At the start of block fb every wave
// issues (a) the global -> LDS DMA (global_load_lds_dwordx4, 1 KB per
// instruction) of block fb+1's weights into the other stage and (b) the load
// of block fb+1's input rows into registers (the B-spline table kernels issue
// the DMA one instruction per slot instead); both are waited for by the
// barrier that closes block fb, so their latency hides behind KP slot steps.
// The two stages are separate __shared__ arrays and the block loop is unrolled
// by two, so the compiler can tell that the B-fragment reads of the current
// stage do not depend on the DMA in flight into the other one.
//
// Within a block a wave walks the KP slots without synchronisation: the
// B-fragments of slot s are read from LDS while the basis values of slot s+1
// are generated into the second A-fragment buffer, then the MFMAs of slot s
// run.  Slots are unrolled by two so the fragment buffers and the Chebyshev
// recurrence roles are fixed at compile time; the B-spline table kernels
// (BASIS_BSPLINE_TAB / _TAB0, K = 8) unroll all KP slots, so every slot's
// basis index is a constant.
//
// Two shapes: WAVES = 4 (tile 4*WM x NB*32, two workgroups per CU) and
// WAVES = 8 with WM = 32, NB = 8 (tile 256 x 256, one workgroup of 8 waves
// per CU).  The second halves the basis values a lane generates per MFMA
// (8 values feed 8 MFMAs); its two stages of up to 10 slots x 8 KB fill the
// 160 KB LDS (9 slots for the RBF and B-spline table kernels, whose lookup
// tables also live in LDS).
//
// KS > 1 (4-wave Chebyshev tiles, small problems): the workgroup holds KS wave
// groups of WAVES waves on the same output tile.  Group g takes its own
// contiguous run of the split's feature blocks with its own two LDS stages;
// all groups run the same number of rounds (a group past its run only joins
// the barrier), so the block barrier stays workgroup-wide.  At the end groups
// 1 .. KS-1 write their accumulators into the then idle stages and group 0
// adds them in group order and writes the tile.  With one workgroup per CU
// this gives 4·KS waves per CU instead of 4 and a KS times shorter chain of
// feature blocks per wave, for layers too small to fill the GPU.
//
// Requires KP = K + has_base <= block_slots(WAVES, BASIS) (the launcher checks).
// ---------------------------------------------------------------------------
// emit<KN> of a table generator (BsplineTab) into the A-fragments a
template <int KN, typename G, typename Frag, int RB>
__device__ __forceinline__ void gen_emit(const G& g, Frag (&a)[RB]) {
  g.template emit<KN>(a);
}

__host__ __device__ constexpr int block_slots(int waves, int basis) {
  return waves == 8 && (basis == BASIS_RBF || basis == BASIS_RBF_TABLE || basis == BASIS_RBF_REC ||
                        basis == BASIS_BSPLINE_TAB || basis == BASIS_BSPLINE_TAB0)
             ? 9
             : 10;
}

// VALU instructions of one slot's basis generation per MFMA of that slot
// (scheduling hint): per value 1 fma (Chebyshev), fma + mul + exp2 (RBF),
// 2 multiplies (RBF recurrence), ~6 compares / selects (B-spline) or none
// (B-spline table), plus the packing into 16-bit pairs.
template <int BASIS, int NV, int MFMAS>
constexpr int kValuPerMfma =
    ((BASIS == BASIS_CHEBY || BASIS == BASIS_CHEBY_POST ? 1
      : BASIS == BASIS_BSPLINE                           ? 6
      : BASIS == BASIS_RBF_REC                           ? 2
      : BASIS == BASIS_BSPLINE_TAB || BASIS == BASIS_BSPLINE_TAB0 ? 0
                                                         : 3) *
         NV + NV / 2 +
     MFMAS - 1) / MFMAS;

// Workgroups per CU the block kernel is compiled for (register budget).
__host__ __device__ constexpr int block_min_wgs(int waves, int nb, int ks) {
  return waves == 4 && (ks == 1 || (ks == 2 && nb == 1)) ? 2 : 1;
}

template <typename T, typename TX, typename TY, int BASIS, int WM, int NB, int WAVES, int KS = 1, bool PAIR = false>
__global__ void __launch_bounds__(WAVES * 64 * KS, block_min_wgs(WAVES, NB, KS))
kan_fused_block(const TX* __restrict__ X, long ldx,
                const uint4* __restrict__ Wt, int nob_pad,
                const T* __restrict__ bias,
                TY* __restrict__ Y, long ldy,
                float* __restrict__ Ypart,
                int B, int D_in, int D_out, int m_tiles, int n_tiles,
                int nfb_total, int fb_per_split, int has_base, BasisParams bp) {
  constexpr int RB = WM / 32;           // 32-row blocks per wave
  constexpr int NV = RB * 8;            // inputs held per lane
  constexpr int CPX = Chunks<TX>::CPL;  // uint4 per lane per row block of inputs
  constexpr int SLOT = NB * 64;         // uint4 per slot of the N-tile
  typedef typename Mfma<T>::frag frag;

  constexpr int SLOTS = block_slots(WAVES, BASIS);
  static_assert(KS == 1 || (WAVES == 4 && (BASIS == BASIS_CHEBY || BASIS == BASIS_CHEBY_POST)),
                "wave groups: 4-wave Chebyshev tiles only");
  __shared__ uint4 stage0[KS * SLOTS * SLOT];
  __shared__ uint4 stage1[KS * SLOTS * SLOT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index as a scalar: the compiler cannot see that tid >> 6 is uniform
  // per wave, and would otherwise keep wave-derived loop counters and
  // addresses in vector registers
  const int wave_wg = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = KS > 1 ? wave_wg / WAVES : 0;  // wave group
  const int wave = KS > 1 ? wave_wg - grp * WAVES : wave_wg;
  int m_tile, n_tile;
  tile_of(xcd_remap(blockIdx.x, m_tiles * n_tiles), m_tiles, n_tiles, m_tile, n_tile);
  const int split = blockIdx.y;

  const int row0 = m_tile * (WAVES * WM) + wave * WM;
  const int ob0 = n_tile * NB;
  const int fb_begin = split * fb_per_split;
  const int fb_end = min(nfb_total, fb_begin + fb_per_split);
  const int KP = bp.K + has_base;
  if (fb_end <= fb_begin) return;  // uniform per workgroup (empty split)
  // this wave group's feature blocks [gb, ge), `rounds` block rounds for every group
  const int rounds = KS > 1 ? (fb_end - fb_begin + KS - 1) / KS : fb_end - fb_begin;
  const int gb = KS > 1 ? min(fb_end, fb_begin + grp * rounds) : fb_begin;
  const int ge = KS > 1 ? min(fb_end, gb + rounds) : fb_end;
  uint4* const st0 = stage0 + (KS > 1 ? grp * SLOTS * SLOT : 0);
  uint4* const st1 = stage1 + (KS > 1 ? grp * SLOTS * SLOT : 0);

  // ---- weights: global -> LDS DMA ------------------------------------------
  // Slot s, column block nb of block fb is W'[fb][s][ob0 + nb][lane]: 64 lanes x
  // 16 B contiguous, one DMA instruction.  Instruction j = s*NB + nb of a block
  // is issued by wave j % WAVES and lands at stage[j * 64 + lane].
  const uint4* wtile = Wt + (long)ob0 * 64 + lane;
  auto dma = [&](int fb, uint4* stage) {
    const uint4* src = wtile + (long)fb * KP * nob_pad * 64;
    for (int j = wave; j < KP * NB; j += WAVES) {
      const int s = j / NB, nb = j - s * NB;
      __builtin_amdgcn_global_load_lds(src + ((long)s * nob_pad + nb) * 64,
                                       (__attribute__((address_space(3))) void*)(stage + j * 64), 16, 0, 0);
    }
  };
  auto bread = [&](frag (&b)[NB], const uint4* stage, int s) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      uint4 u = stage[(s * NB + nb) * 64 + lane];
      b[nb] = *reinterpret_cast<frag*>(&u);
    }
  };

  // ---- inputs: lane holds x[row0 + rb*32 + lane%32][fb*16 + 8*(lane/32) + j] --
  uint4 xr[RB][CPX];
  auto xload = [&](int fbx) {
    const int f0 = fbx * 16 + 8 * (lane >> 5);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = row0 + rb * 32 + (lane & 31);
      const bool ok = (row < B) && (f0 < D_in);
      const uint4* p = reinterpret_cast<const uint4*>(X + (long)row * ldx + f0);
#pragma unroll
      for (int c = 0; c < CPX; ++c) xr[rb][c] = ok ? p[c] : make_uint4(0, 0, 0, 0);
    }
  };
  // unpack to fp32; inputs at or beyond D_in read as 0 whatever the padding holds
  auto xunpack = [&](int fbx, float* xf) {
    const int f0 = fbx * 16 + 8 * (lane >> 5);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int c = 0; c < CPX; ++c) {
        const uint4 u = xr[rb][c];
        if constexpr (sizeof(TX) == 4) {
          xf[rb * 8 + c * 4 + 0] = __uint_as_float(u.x);
          xf[rb * 8 + c * 4 + 1] = __uint_as_float(u.y);
          xf[rb * 8 + c * 4 + 2] = __uint_as_float(u.z);
          xf[rb * 8 + c * 4 + 3] = __uint_as_float(u.w);
        } else {
          const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            TX lo, hi;
            const unsigned short l16 = (unsigned short)(w[q] & 0xffffu), h16 = (unsigned short)(w[q] >> 16);
            __builtin_memcpy(&lo, &l16, 2);
            __builtin_memcpy(&hi, &h16, 2);
            xf[rb * 8 + 2 * q] = to_f32(lo);
            xf[rb * 8 + 2 * q + 1] = to_f32(hi);
          }
        }
      }
    // only the last feature block can reach past D_in: a wave-uniform test
    // keeps the per-lane masking out of every other block
    if ((fbx + 1) * 16 > D_in) {
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (f0 + (j & 7) >= D_in) xf[j] = 0.0f;
    }
  };
  auto pack = [&](frag (&a)[RB], const float* v) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int j = 0; j < 8; ++j) a[rb][j] = from_f32<T>(v[rb * 8 + j]);
  };

  floatx16 acc[RB][NB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[rb][nb][r] = 0.0f;

  // ---- prologue: the group's first block in its stage 0 and registers -------
  // B-spline table kernels: HB = has_base at compile time
  constexpr bool kTab = BASIS == BASIS_BSPLINE_TAB || BASIS == BASIS_BSPLINE_TAB0;
  typedef typename std::conditional<kTab, BsplineTab<T, NV>, BasisGen<BASIS, NV>>::type Gen;
  Gen gen;
  __shared__ uint4 bs_sel[kBsplineTabG];  // table kernels: perm selectors per span
  if constexpr (kTab) {
    if (tid < kBsplineTabG)
      bs_sel[tid] = make_uint4(bspline_tab_selector(tid, 0), bspline_tab_selector(tid, 1),
                               bspline_tab_selector(tid, 2), bspline_tab_selector(tid, 3));
  }
  if constexpr (BASIS == BASIS_RBF_TABLE) {
    // scaled centres s*c_k, entry K = 0 (read by the unused step after a
    // block's last slot)
    __shared__ float rbf_tab[kMaxK + 1];
    if (tid <= bp.K) rbf_tab[tid] = tid < bp.K ? bp.rbf_sc[tid] : 0.0f;
    gen.tab = rbf_tab;
  }
  // PAIR: two feature blocks per stage (the launcher checks 2 KP <= SLOTS): one
  // barrier per two blocks, the DMA of block fb + 2 issued in block fb into the
  // same half of the other stage.  Same arithmetic in the same order as one
  // block per stage.  A separate instantiation, so that the one-block kernels
  // keep their registers and schedule.
  static_assert(!PAIR || (KS == 1 && !kTab), "block pairs: one wave group, slot-loop kernels");
  if (KS == 1 || gb < ge) {
    dma(gb, st0);
    if constexpr (PAIR) {
      if (gb + 1 < ge) dma(gb + 1, st0 + KP * SLOT);
    }
    xload(gb);
  }
  __syncthreads();
  // kHoist (RBF): the B fragments in one register set per slot parity and the
  // read addresses of a slot pair hoisted (see the slot loop).  Measured on
  // the 16384 x 1024 -> 1024 shapes: RBF +2.3 %, Chebyshev -1.7 % (its
  // per-slot fence then leaves every read behind the slot's MFMAs); the
  // generic B-spline and the (64,4) kernels sit at the 256-register limit.
  constexpr bool kHoist = BASIS == BASIS_RBF_REC || BASIS == BASIS_RBF_TABLE;
  frag af[2][RB], bfr[kHoist ? 2 : 1][NB];
  // One slot s of parity P, a single basic block: the MFMAs of slot s (on
  // af[P], bf) are interleaved with the basis values of slot s+1 (into
  // af[P^1]; the last slot of a block computes one unused extra) and the
  // B-fragment reads of slot s+1 (clamped to the block).  Each bf[nb] is
  // re-read as soon as its last MFMA has issued.
  // gen_next(af[P ^ 1]) produces the A-fragment of slot s + 1; sn = the slot
  // whose B-fragments are read (s + 1 clamped to the block).
  // Table kernels spread the weight DMA of the next block over the slots: the
  // wave's DMA instruction si (of KP, since NB == WAVES) is issued in slot si
  // from dsrc into ddst, set at the block start.  The other kernels issue it all
  // at the block start (measured: the spread gains 2 % on the fully unrolled
  // table kernels and loses 1-3 % in the slot loop of the others).
  const uint4* dsrc = wtile;
  uint4* ddst = st1;
  auto dma_one = [&](int si) __attribute__((always_inline)) {
    static_assert(!kTab || (NB == WAVES), "one DMA instruction per wave and slot");
    const int j = wave + si * WAVES;
    const int ss = j / NB, nb = j - ss * NB;
    __builtin_amdgcn_global_load_lds(dsrc + ((long)ss * nob_pad + nb) * 64,
                                     (__attribute__((address_space(3))) void*)(ddst + j * 64), 16, 0, 0);
  };
  // Reads of slot sn's B fragments: cur[(sn * NB + nb) * 64 + lane], or with
  // off >= 0 cur[off + nb * 64] (the slot loop passes cur = this lane's chunk of
  // slot sn, precomputed, and off = 0).
  auto slot_core = [&](const uint4* cur, int si, int sn, auto PP, auto&& gen_next, int off = -1)
      __attribute__((always_inline)) {
    constexpr int P = decltype(PP)::value;
    frag(&bcur)[NB] = bfr[kHoist ? P : 0];
    frag(&bnext)[NB] = bfr[kHoist ? P ^ 1 : 0];
    if constexpr (kTab) dma_one(si);
    gen_next(af[P ^ 1]);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][nb] = Mfma<T>::mma(af[P][rb], bcur[nb], acc[rb][nb]);
      uint4 u = off >= 0 ? cur[off + nb * 64] : cur[(sn * NB + nb) * 64 + lane];
      bnext[nb] = *reinterpret_cast<frag*>(&u);
    }
    // issue order: per column block, RB MFMAs each followed by a share of the
    // basis-generation VALU work, then that block's next B-fragment read.
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma<BASIS, NV, RB * NB>, 0);  // VALU
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                     // DS read
    }
    // Chebyshev: nothing crosses into the next slot (otherwise the scheduler
    // sinks this slot's B-fragment reads into the next one, which then waits
    // on LDS latency before its MFMAs; measured 3-4 % faster).  The RBF and
    // B-spline schedules measured better without the fence.
    if constexpr (BASIS == BASIS_CHEBY_POST) __builtin_amdgcn_sched_barrier(0);
  };
  auto slot = [&](const uint4* cur, int s, auto PP, int off = -1) {
    constexpr int P = decltype(PP)::value;
    slot_core(cur, s, min(s + 1, KP - 1), PP, [&](frag(&a)[RB]) __attribute__((always_inline)) {
      if constexpr (!kTab) {
        float v[NV];
        gen.template step<P ^ 1>(s + 1 - has_base, bp, v);
        pack(a, v);
      }
    }, off);
  };
  // Table kernels: K = 8 and HB = has_base known at compile time, so every
  // slot's basis index is a constant and emit<k> reads fixed table registers.
  auto tab_slots = [&](const uint4* cur) __attribute__((always_inline)) {
    constexpr int HB = BASIS == BASIS_BSPLINE_TAB ? 1 : 0;
    constexpr int KPC = kBsplineTabG + 3 + HB;
    static_for<0, KPC>([&](auto SC) __attribute__((always_inline)) {
      constexpr int sc = decltype(SC)::value;
      constexpr int kn = sc + 1 - HB;  // basis of slot sc + 1
      slot_core(cur, sc, sc + 1 < KPC ? sc + 1 : KPC - 1, std::integral_constant<int, sc & 1>{},
                [&](frag(&a)[RB]) __attribute__((always_inline)) {
        if constexpr (kTab && kn < kBsplineTabG + 3) gen_emit<kn>(gen, a);
      });
      // keep the unrolled slots apart, as the loop's basic blocks keep them for
      // the other bases: hoisting later slots' B-fragment reads costs registers
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // ahead: the block whose weights this one copies into nxt (fb + 1, or fb + 2
  // with two blocks per stage)
  auto block = [&](int fb, const uint4* cur, uint4* nxt, int ahead) {
    float xf[NV];
    xunpack(fb, xf);
    if (fb + 1 < ge) xload(fb + 1);
    if constexpr (kTab) {
      // the last block reloads its own weights into the idle stage (in bounds,
      // branch-free; waited for by the closing barrier like the others)
      dsrc = wtile + (long)min(fb + 1, ge - 1) * KP * nob_pad * 64;
      ddst = nxt;
    } else if (fb + ahead < ge) {
      dma(fb + ahead, nxt);
    }
    if constexpr (kTab) {
      // the table first: its selector reads and temporaries die before the
      // first slot's B-fragments occupy their 32 registers
      gen.begin(xf, bp, bs_sel);
      __builtin_amdgcn_sched_barrier(0);
      bread(bfr[0], cur, 0);
      // the reads issue here: in the region of slot 0 the scheduler placed
      // each just before its MFMA, which then waited for it
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (BASIS == BASIS_BSPLINE_TAB) {
        float v[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = silu_f32(xf[i]);
        pack(af[0], v);
      } else {
        gen_emit<0>(gen, af[0]);
      }
      tab_slots(cur);
    } else {
      bread(bfr[0], cur, 0);
      // basis k is emitted at slot k + has_base: basis 0 lands at parity has_base
      gen.begin(xf, bp, has_base != 0);
      {
        float v[NV];
        if (has_base) {
#pragma unroll
          for (int i = 0; i < NV; ++i) v[i] = silu_f32(xf[i]);
        } else {
          gen.template step<0>(0, bp, v);
        }
        pack(af[0], v);
      }
      // slot pairs as one branch-free basic block; an odd last slot is peeled
      int s = 0;
      for (; s + 1 < KP; s += 2) {
        if constexpr (kHoist) {
          // the two slots' read addresses in a scheduling region of their own:
          // inside the slots' region the scheduler placed that VALU late, and
          // every B-fragment read of the pair's first slot behind it, so the
          // second slot waited on LDS latency before every other MFMA
          const uint4* rd0 = cur + min(s + 1, KP - 1) * NB * 64 + lane;
          const uint4* rd1 = cur + min(s + 2, KP - 1) * NB * 64 + lane;
          __builtin_amdgcn_sched_barrier(0);
          slot(rd0, s, std::integral_constant<int, 0>{}, 0);
          slot(rd1, s + 1, std::integral_constant<int, 1>{}, 0);
        } else {
          slot(cur, s, std::integral_constant<int, 0>{});
          slot(cur, s + 1, std::integral_constant<int, 1>{});
        }
      }
      if (s < KP) slot(cur, s, std::integral_constant<int, 0>{});
    }
  };
  // each block ends with the barrier that waits for its successor's DMA and
  // input loads and frees its stage
  if constexpr (KS == 1) {
    if constexpr (PAIR) {
      uint4* const st0b = st0 + KP * SLOT;
      uint4* const st1b = st1 + KP * SLOT;
      for (int fb = fb_begin; fb < fb_end; fb += 4) {
        block(fb, st0, st1, 2);
        if (fb + 1 < fb_end) block(fb + 1, st0b, st1b, 2);
        __syncthreads();
        if (fb + 2 < fb_end) {
          block(fb + 2, st1, st0, 2);
          if (fb + 3 < fb_end) block(fb + 3, st1b, st0b, 2);
          __syncthreads();
        }
      }
    } else {
      for (int fb = fb_begin; fb < fb_end; fb += 2) {
        block(fb, st0, st1, 1);
        __syncthreads();
        if (fb + 1 < fb_end) {
          block(fb + 1, st1, st0, 1);
          __syncthreads();
        }
      }
    }
  } else {
    // every group runs `rounds` rounds; a group past its run only joins the barrier
    for (int it = 0; it < rounds; it += 2) {
      if (gb + it < ge) block(gb + it, st0, st1, 1);
      __syncthreads();
      if (it + 1 < rounds) {
        if (gb + it + 1 < ge) block(gb + it + 1, st1, st0, 1);
        __syncthreads();
      }
    }
    // groups 1 .. KS-1 hand their accumulators to group 0 through the idle
    // stages (lane-contiguous, conflict-free); group 0 adds them in group order
    constexpr int NACC = RB * NB * 16;
    constexpr int GRP_FLOATS = WAVES * NACC * 64;
    constexpr int PER_STAGE = KS * SLOTS * SLOT * 4 / GRP_FLOATS;  // groups per stage array
    static_assert(2 * PER_STAGE >= KS - 1, "wave-group reduction does not fit the stages");
    auto red_of = [&](int g) -> float* {  // g = 1 .. KS-1
      const int i = g - 1;
      float* base = reinterpret_cast<float*>(i < PER_STAGE ? stage0 : stage1);
      const int j = i < PER_STAGE ? i : i - PER_STAGE;
      return base + (j * WAVES + wave) * NACC * 64 + lane;
    };
    if (grp > 0) {
      float* r = red_of(grp);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int q = 0; q < 16; ++q) r[((rb * NB + nb) * 16 + q) * 64] = acc[rb][nb][q];
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int g = 1; g < KS; ++g) {
      const float* r = red_of(g);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int q = 0; q < 16; ++q) acc[rb][nb][q] += r[((rb * NB + nb) * 16 + q) * 64];
    }
  }

  // ---- epilogue -------------------------------------------------------------
  // acc register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  const int rbase = row0 + 4 * (lane >> 5);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int col = (ob0 + nb) * 32 + (lane & 31);
    if (col < D_out) {
      if (Ypart != nullptr) {
        float* out = Ypart + ((long)split * B + rbase) * D_out + col;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dr = rb * 32 + 8 * (r >> 2) + (r & 3);
            if (rbase + dr < B) out[(long)dr * D_out] = acc[rb][nb][r];
          }
      } else {
        const float bcol = bias != nullptr ? to_f32(bias[col]) : 0.0f;
        TY* out = Y + (long)rbase * ldy + col;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dr = rb * 32 + 8 * (r >> 2) + (r & 3);
            // y is written once and not read here: non-temporal stores keep
            // L2 for the inputs and weights (measured 0.5 % on the 16384 x
            // 1024 -> 1024 shapes)
            if (rbase + dr < B)
              __builtin_nontemporal_store(from_f32<TY>(acc[rb][nb][r] + bcol), out + (long)dr * ldy);
          }
      }
    }
  }
}

// Split reduction: y = sum_split part[split] + bias, converted to T.
template <typename T, typename TY>
__global__ void kan_split_finalize(const float* __restrict__ part, int splits, const T* __restrict__ bias,
                                   TY* __restrict__ Y, long ldy, int B, int D_out) {
  long n = (long)B * D_out;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (long)gridDim.x * blockDim.x) {
    int row = (int)(idx / D_out), col = (int)(idx - (long)row * D_out);
    float s = bias ? to_f32(bias[col]) : 0.0f;
    // splits in order, loaded 8 at a time: one memory round trip per 8
    // splits instead of one per split
    for (int k0 = 0; k0 < splits; k0 += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = k0 + u < splits ? part[(long)(k0 + u) * n + idx] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k0 + u < splits) s += v[u];
    }
    Y[(long)row * ldy + col] = from_f32<TY>(s);
  }
}

// The same reduction for 4 consecutive columns per thread (D_out and ldy
// multiples of 4, Y aligned to 4 elements): 16-byte partial loads and one
// vector store, the same sum order per element.
template <typename T, typename TY>
__global__ void kan_split_finalize4(const float4* __restrict__ part, int splits, const T* __restrict__ bias,
                                    TY* __restrict__ Y, long ldy, int B, int D_out) {
  const long n4 = (long)B * D_out / 4;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (long)gridDim.x * blockDim.x) {
    const long idx = 4 * i;
    const int row = (int)(idx / D_out), col = (int)(idx - (long)row * D_out);
    float s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = bias ? to_f32(bias[col + j]) : 0.0f;
    for (int k0 = 0; k0 < splits; k0 += 8) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = k0 + u < splits ? part[(long)(k0 + u) * n4 + i] : make_float4(0, 0, 0, 0);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k0 + u < splits) {
          s[0] += v[u].x;
          s[1] += v[u].y;
          s[2] += v[u].z;
          s[3] += v[u].w;
        }
    }
    TY* out = Y + (long)row * ldy + col;
    if constexpr (sizeof(TY) == 4) {
      *reinterpret_cast<float4*>(out) = make_float4(s[0], s[1], s[2], s[3]);
    } else {
      TY h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = from_f32<TY>(s[j]);
      uint2 u;
      __builtin_memcpy(&u, h, 8);
      *reinterpret_cast<uint2*>(out) = u;
    }
  }
}

// Repack raw weights W[D_out][D_in*K] (k fastest) and W_base[D_out][D_in], of
// element type S, into the tiled layout W'[fb][s][ob][chunk][lane][e] of type T
// (see kans_common.h), converting S -> T with round-to-nearest-even; zero
// padding for o >= D_out and i >= D_in.
template <typename S, typename T>
__global__ void kan_repack_weights(const S* __restrict__ W, const S* __restrict__ Wb, uint4* __restrict__ Wt,
                                   int D_in, int D_out, int K, int has_base, int nfb, int nob_pad) {
  constexpr int CPL = Chunks<T>::CPL;
  constexpr int EPC = 16 / (int)sizeof(T);
  const int KP = K + has_base;
  const long total = (long)nfb * KP * nob_pad * CPL * 64;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (long)gridDim.x * blockDim.x) {
    long r = idx;
    const int lane = (int)(r % 64); r /= 64;
    const int chunk = (int)(r % CPL); r /= CPL;
    const int ob = (int)(r % nob_pad); r /= nob_pad;
    const int s = (int)(r % KP); r /= KP;
    const int fb = (int)r;
    const int o = ob * 32 + (lane & 31);
    const int ibase = fb * 16 + 8 * (lane >> 5) + chunk * EPC;
    T vals[EPC];
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const int i = ibase + e;
      float w = 0.0f;
      if (o < D_out && i < D_in) {
        if (has_base && s == 0) w = to_f32(Wb[(long)o * D_in + i]);
        else w = to_f32(W[((long)o * D_in + i) * K + (s - has_base)]);
      }
      vals[e] = from_f32<T>(w);
    }
    Wt[idx] = *reinterpret_cast<uint4*>(vals);
  }
}

template <typename S, typename T>
__global__ void kan_convert(const S* __restrict__ src, T* __restrict__ dst, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    dst[i] = from_f32<T>(to_f32(src[i]));
}

// ---------------------------------------------------------------------------
// Host-side launch.
// ---------------------------------------------------------------------------


int block_waves(bool half, int basis, int wm, int nb, int KP);

template <typename T, typename TX, typename TY, int BASIS, int WM, int NB>
static hipError_t launch_dense_t(const DenseLaunch& L, hipStream_t st) {
  const int m_tiles = (L.B + 4 * WM - 1) / (4 * WM);
  const int nob = (L.D_out + 31) / 32;
  const int n_tiles = (nob + NB - 1) / NB;
  const int fbps = (L.nfb + L.splits - 1) / L.splits;
  const int splits = (L.nfb + fbps - 1) / fbps;
  dim3 grid(m_tiles * n_tiles, splits);
  float* part = splits > 1 ? L.part : nullptr;
  // Kernel choice for 16-bit layers whose feature block fits one LDS stage:
  //   Chebyshev, tiles up to NB = 4        -> block kernel, 4 waves;
  //   RBF / B-spline, tile (32,8)          -> block kernel, 8 waves (256 x 256);
  // everything else (fp32, other tiles, larger K) -> the per-slot kernel.
  const int waves = block_waves(sizeof(T) == 2, BASIS, WM, NB, L.bp.K + L.has_base);
  constexpr bool kBlock4 = sizeof(T) == 2 && BASIS == BASIS_CHEBY && NB <= 4;
  constexpr bool kBlock8 = sizeof(T) == 2 && WM == 32 && NB == 8;
  if (waves == 4) {
    if constexpr (kBlock4) {
      constexpr int BB = BASIS == BASIS_CHEBY ? BASIS_CHEBY_POST : BASIS;
      auto go = [&](auto KSC) {
        constexpr int KS = decltype(KSC)::value;
        hipLaunchKernelGGL((kan_fused_block<T, TX, TY, BB, WM, NB, 4, KS>), grid, dim3(256 * KS), 0, st,
                           (const TX*)L.X, L.ldx, (const uint4*)L.Wt, L.nob_pad, (const T*)L.bias, (TY*)L.Y, L.ldy,
                           part, L.B, L.D_in, L.D_out, m_tiles, n_tiles, L.nfb, fbps, L.has_base, L.bp);
      };
      // wave groups (block_wave_groups_ok): 2 on (32,1) and (32,4), 4 on (32,1)
      if constexpr (WM == 32 && NB == 1) {
        if (L.ks == 4) go(std::integral_constant<int, 4>{});
        else if (L.ks == 2) go(std::integral_constant<int, 2>{});
        else go(std::integral_constant<int, 1>{});
      } else if constexpr (WM == 32 && NB == 4) {
        if (L.ks == 2) go(std::integral_constant<int, 2>{});
        else go(std::integral_constant<int, 1>{});
      } else {
        go(std::integral_constant<int, 1>{});
      }
    }
  } else if (waves == 8) {
    if constexpr (kBlock8) {
      const int m_tiles8 = (L.B + 8 * WM - 1) / (8 * WM);
      auto go = [&](auto BBC) {
        constexpr int BB = decltype(BBC)::value;
        auto launch = [&](auto PC) {
          hipLaunchKernelGGL((kan_fused_block<T, TX, TY, BB, WM, NB, 8, 1, decltype(PC)::value>),
                             dim3(m_tiles8 * n_tiles, splits), dim3(512), 0, st, (const TX*)L.X, L.ldx,
                             (const uint4*)L.Wt, L.nob_pad, (const T*)L.bias, (TY*)L.Y, L.ldy, part, L.B, L.D_in,
                             L.D_out, m_tiles8, n_tiles, L.nfb, fbps, L.has_base, L.bp);
        };
        // two feature blocks per LDS stage (Chebyshev, K + has_base <= 5)
        if constexpr (BB == BASIS_CHEBY_POST) {
          if (L.pair && 2 * (L.bp.K + L.has_base) <= block_slots(8, BB)) {
            launch(std::true_type{});
            return;
          }
        }
        launch(std::false_type{});
      };
      if constexpr (BASIS == BASIS_RBF) {
        // uniform centres: the two-multiply recurrence; otherwise exp2 per value
        if (L.bp.rbf_rec) go(std::integral_constant<int, BASIS_RBF_REC>{});
        else go(std::integral_constant<int, BASIS_RBF_TABLE>{});
      } else if constexpr (BASIS == BASIS_BSPLINE) {
        // G = 5: per-input basis table (one v_perm per two values per slot)
        if (L.bp.grid_size == kBsplineTabG && L.has_base) go(std::integral_constant<int, BASIS_BSPLINE_TAB>{});
        else if (L.bp.grid_size == kBsplineTabG) go(std::integral_constant<int, BASIS_BSPLINE_TAB0>{});
        else go(std::integral_constant<int, BASIS_BSPLINE>{});
      } else {
        go(std::integral_constant<int, BASIS == BASIS_CHEBY ? BASIS_CHEBY_POST : BASIS>{});
      }
    }
  } else {
    hipLaunchKernelGGL((kan_fused_dense<T, TX, TY, BASIS, WM, NB>), grid, dim3(kThreads), 0, st, (const TX*)L.X,
                       L.ldx, (const uint4*)L.Wt, L.nob_pad, (const T*)L.bias, (TY*)L.Y, L.ldy, part, L.B, L.D_in,
                       L.D_out, m_tiles, n_tiles, L.nfb, fbps, L.has_base, L.bp);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (splits > 1) {
    const long n = (long)L.B * L.D_out;
    if (L.D_out % 4 == 0 && L.ldy % 4 == 0 && ((uintptr_t)L.Y % (4 * sizeof(TY))) == 0) {
      const int blocks = (int)std::min<long>((n / 4 + 255) / 256, 4096);
      hipLaunchKernelGGL((kan_split_finalize4<T, TY>), dim3(blocks), dim3(256), 0, st, (const float4*)part, splits,
                         (const T*)L.bias, (TY*)L.Y, L.ldy, L.B, L.D_out);
    } else {
      const int blocks = (int)std::min<long>((n + 255) / 256, 4096);
      hipLaunchKernelGGL((kan_split_finalize<T, TY>), dim3(blocks), dim3(256), 0, st, part, splits,
                         (const T*)L.bias, (TY*)L.Y, L.ldy, L.B, L.D_out);
    }
    e = hipGetLastError();
  }
  return e;
}

// Workgroup waves of the block kernel for this configuration, 0 when the
// per-slot kernel runs (the routing of launch_dense_t).
int block_waves(bool half, int basis, int wm, int nb, int KP) {
  if (!half) return 0;
  if (basis == BASIS_CHEBY && nb <= 4 && KP <= block_slots(4, basis)) return 4;
  if (wm == 32 && nb == 8 && KP <= block_slots(8, basis)) return 8;
  return 0;
}

// Instantiated tile configurations (WM rows per wave, NB 32-column blocks):
// (64,4) (32,8) (32,4) (32,1); at most 128 fp32 accumulators per lane so two
// workgroups (8 waves) stay resident per CU.  (32,8) halves the basis values a
// lane generates per MFMA relative to (64,4).  Keep in sync with
// dense_config_supported().
template <typename T, typename TX, typename TY, int BASIS>
static hipError_t launch_dense_cfg(const DenseLaunch& L, hipStream_t st) {
  if (L.wm == 64 && L.nb == 4) return launch_dense_t<T, TX, TY, BASIS, 64, 4>(L, st);
  if (L.wm == 32 && L.nb == 8) return launch_dense_t<T, TX, TY, BASIS, 32, 8>(L, st);
  if (L.wm == 32 && L.nb == 4) return launch_dense_t<T, TX, TY, BASIS, 32, 4>(L, st);
  if (L.wm == 32 && L.nb == 1) return launch_dense_t<T, TX, TY, BASIS, 32, 1>(L, st);
  return hipErrorInvalidValue;
}

// Wave groups per workgroup the 4-wave block kernel is instantiated with for a
// tile (KS = 1 always).  Keep in sync with launch_dense_t.
bool block_wave_groups_ok(int wm, int nb, int ks) {
  return ks == 1 || (wm == 32 && ((nb == 1 && (ks == 2 || ks == 4)) || (nb == 4 && ks == 2)));
}

bool dense_config_supported(int wm, int nb) {
  return (wm == 64 && nb == 4) || (wm == 32 && (nb == 8 || nb == 4 || nb == 1));
}

template <typename T, typename TX, typename TY>
static hipError_t launch_dense_io(const DenseLaunch& L, hipStream_t st) {
  switch (L.basis) {
    case BASIS_CHEBY: return launch_dense_cfg<T, TX, TY, BASIS_CHEBY>(L, st);
    case BASIS_RBF: return launch_dense_cfg<T, TX, TY, BASIS_RBF>(L, st);
    default: return launch_dense_cfg<T, TX, TY, BASIS_BSPLINE>(L, st);
  }
}

// x_dtype / y_dtype: the layer dtype or DT_F32 (fp32 activations around a 16-bit layer).
template <typename T>
static hipError_t launch_dense_type(const DenseLaunch& L, hipStream_t st) {
  const bool xf = L.x_dtype == DT_F32 && L.dtype != DT_F32;
  const bool yf = L.y_dtype == DT_F32 && L.dtype != DT_F32;
  if (!xf && !yf) return launch_dense_io<T, T, T>(L, st);
  if constexpr (sizeof(T) == 2) {
    if (xf && yf) return launch_dense_io<T, float, float>(L, st);
    if (xf) return launch_dense_io<T, float, T>(L, st);
    return launch_dense_io<T, T, float>(L, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_dense(const DenseLaunch& L, hipStream_t st) {
  switch (L.dtype) {
    case DT_F16: return launch_dense_type<_Float16>(L, st);
    case DT_BF16: return launch_dense_type<__bf16>(L, st);
    default: return launch_dense_type<float>(L, st);
  }
}

template <typename S, typename T>
static hipError_t repack_t(const void* W, const void* Wb, void* Wt, int D_in, int D_out, int K, int has_base,
                           int nfb, int nob_pad, hipStream_t st) {
  const int KP = K + has_base;
  long total = (long)nfb * KP * nob_pad * Chunks<T>::CPL * 64;
  int blocks = (int)std::min<long>((total + 255) / 256, 16384);
  hipLaunchKernelGGL((kan_repack_weights<S, T>), dim3(blocks), dim3(256), 0, st, (const S*)W, (const S*)Wb,
                     (uint4*)Wt, D_in, D_out, K, has_base, nfb, nob_pad);
  return hipGetLastError();
}

// src_dtype: element type of W / Wb (same as dtype, or DT_F32 for a converting upload).
hipError_t launch_repack(int src_dtype, int dtype, const void* W, const void* Wb, void* Wt, int D_in, int D_out,
                         int K, int has_base, int nfb, int nob_pad, hipStream_t st) {
  if (src_dtype == dtype) {
    switch (dtype) {
      case DT_F16: return repack_t<_Float16, _Float16>(W, Wb, Wt, D_in, D_out, K, has_base, nfb, nob_pad, st);
      case DT_BF16: return repack_t<__bf16, __bf16>(W, Wb, Wt, D_in, D_out, K, has_base, nfb, nob_pad, st);
      default: return repack_t<float, float>(W, Wb, Wt, D_in, D_out, K, has_base, nfb, nob_pad, st);
    }
  }
  if (src_dtype != DT_F32) return hipErrorInvalidValue;
  switch (dtype) {
    case DT_F16: return repack_t<float, _Float16>(W, Wb, Wt, D_in, D_out, K, has_base, nfb, nob_pad, st);
    case DT_BF16: return repack_t<float, __bf16>(W, Wb, Wt, D_in, D_out, K, has_base, nfb, nob_pad, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_convert(int src_dtype, int dtype, const void* src, void* dst, long n, hipStream_t st) {
  int blocks = (int)std::min<long>((n + 255) / 256, 4096);
  if (src_dtype != DT_F32 || dtype == DT_F32) return hipErrorInvalidValue;
  if (dtype == DT_F16)
    hipLaunchKernelGGL((kan_convert<float, _Float16>), dim3(blocks), dim3(256), 0, st, (const float*)src,
                       (_Float16*)dst, n);
  else
    hipLaunchKernelGGL((kan_convert<float, __bf16>), dim3(blocks), dim3(256), 0, st, (const float*)src,
                       (__bf16*)dst, n);
  return hipGetLastError();
}

}  // namespace kans
