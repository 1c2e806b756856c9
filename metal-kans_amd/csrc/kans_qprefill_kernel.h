// Fused prefill (large-batch) forward of Chebyshev KAN layers whose weights are
// held in the reference's packed INT8 / INT4 (group 64, scale + bias) or
// ternary (group 32, absmean scale) formats, and of the GatedKAN gate|up pair
// with its SwiGLU epilogue.
//
//   y[b,o] = bias[o] + sum_i SiLU(x[b,i]) Wb[o,i] + sum_{i,k} T_k(clamp x[b,i]) W[o,i*K+k]
//   W = q*s + b per group (quantization.py:13-99,136-148) or t*s (:191-246,275-286)
//
// The reference dequantizes to fp32 on the host and runs the fp32 forward
// (quantization.py:152-188, gated_kan.py:86-138).  Here the weights stay packed
// in HBM and are decoded on their way into the MFMA B-tiles, so a forward moves
// the packed bytes (INT4: 0.53 B per weight with its parameters, ternary 0.28 B)
// instead of 2-4 bytes per weight.
//
// Work decomposition: the 256 x 256 tile of the fp16 block kernel
// (kan_fused_block, WAVES = 8, WM = 32, NB = 8): each wave owns 32 rows x 256
// columns and walks feature blocks of 16 inputs x KP = K + has_base slots,
// generating the Chebyshev / SiLU values of its rows in registers (the A
// fragments) and multiplying them by B fragments read from LDS.  What differs
// is how a feature block's weights reach LDS: instead of a DMA of fp16 tiles,
// wave w decodes column block w of the N-tile itself.  For the KP slots of
// block fb+1 its lanes hold the 8-code chunks (loaded one block ahead into a
// two-deep register ring) and their group parameters; in slot s of block fb
// each lane turns the chunk of slot s into 8 fp16 weights and writes them with
// one ds_write_b128 to the idle LDS stage, interleaved with the MFMAs of slot s.
//   INT4: nibbles -> fp16 (1024 + q) / (64 + q) with two v_and_or_b32 per dword
//         pair (fp16 magic exponents), then v_fma_mix: fp16(V*s + (b - off*s));
//   INT8: bytes -> fp16 (1024 + q) with v_perm_b32, then v_fma_mix;
//   ternary: codes -> {-1, 0, +1} fp16 with a v_perm_b32 table, then a packed
//         fp16 multiply by fp16(s) (exact: fp16(t*s) = t*fp16(s)).
// The affine weights are computed in fp32 with one rounding (fma) from the
// fp32 parameters and then rounded once to fp16, the operand type of the MFMA.
//
// gate|up (grp = 4): column blocks 0..3 of an N-tile are gate columns
// 128 n .. 128 n + 127, blocks 4..7 the same up columns, so the epilogue finds
// gate and up of one output in the same lane and register and writes
// hidden = SiLU(gate) * up (the +-20 clip of gated_kan.py:15-16) without the
// gate / up activations ever reaching memory.
//
// This header holds the kernel template and its launch (qp_run<QT, HB>); each
// weight format and base flag instantiates it in a translation unit of its
// own (kans_qprefill_{int4,int8,tern}_b{0,1}.hip), so the instantiations
// compile in parallel.  kans_qprefill.hip holds the split reduction, the re-tiling
// kernels and the host launch.
#pragma once
#include "kans_common.h"
#include "kans_api_internal.h"
#include "kans_tile.h"
#include "kans_qgemv.h"
#include "kans_qprefill.h"
#include <algorithm>

namespace kans {

namespace {

constexpr int kQWaves = 8, kQNB = 8, kQThreads = 512;
// code e of an INT4 chunk dword sits at bit kInt4Pos[e]: the fp16 pairs
// (e0,e1), (e4,e5) are the low nibbles of each 16-bit half of w and w >> 8,
// (e2,e3), (e6,e7) the second nibbles
__host__ __device__ constexpr int int4_pos(int e) { return (e & 1) * 16 + (e >> 1) * 4; }

// Decode constants in VGPRs (opaque to constant folding, so the compiler selects
// one v_and_or_b32 per pair; see UnpackConsts in kans_qgemv.hip).
// Only the constants of format QT are materialised (each costs a register).
template <int QT>
struct DqConsts {
  unsigned m_lo = 0x000F000Fu, m_hi = 0x00F000F0u;
  unsigned c1024 = 0x64006400u;  // fp16 1024.0 in both halves
  unsigned c64 = 0x54005400u;    // fp16 64.0
  unsigned c64x4 = 0x64646464u;  // high byte of fp16 1024 + q for v_perm
  unsigned t_mask = 0x03000300u, t_zero = 0x000C000Cu;
  __device__ __forceinline__ void init() {
    if constexpr (QT == Q_INT4) asm volatile("" : "+v"(m_lo), "+v"(m_hi), "+v"(c1024), "+v"(c64));
    else if constexpr (QT == Q_INT8) asm volatile("" : "+v"(c64x4));
    else asm volatile("" : "+v"(t_mask), "+v"(t_zero));
  }
};

// fp16 pair (V0, V1) -> (fp16(V0*s0 + off0), fp16(V1*s1 + off1)), each one fma
// in fp32 with an fp16 source and an fp16 result: v_fma_mixlo_f16 writes the
// low half, v_fma_mixhi_f16 the high half of the same register (the compiler
// builds the pair from two mixlo results, a shift and an or instead).
// op_sel_hi:[1,0,0] reads src0 as fp16 (op_sel picks its half), s and off as
// fp32.
__device__ __forceinline__ unsigned fmix2(unsigned u, float s0, float off0, float s1, float off1) {
  unsigned r;
  asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(u), "v"(s0), "v"(off0));
  asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(r) : "v"(u), "v"(s1), "v"(off1));
  return r;
}

// Decode parameters of the NG groups a half-block meets (set once per feature
// block): affine scale, bias - 1024 s and bias - 64 s; ternary fp16(scale) in
// both halves.
template <int NG>
struct DqGroups {
  float s[NG], b1024[NG], b64[NG];
  unsigned h[NG];
};
__device__ __forceinline__ unsigned half2_of(float s) {
  const _Float16 h = (_Float16)s;
  unsigned short u;
  __builtin_memcpy(&u, &h, 2);
  return (unsigned)u | ((unsigned)u << 16);
}

// Group of one code: D0 for the lanes of half 0, D1 for half 1 (compile time).
// m0 is all ones in the lanes of half 0 and zero in half 1, opaque to the
// compiler: equal groups cost nothing, different ones one v_bfi_b32 (a select
// on the half was turned into an indexed load of the parameter array, which
// then lived in scratch memory).
template <int D0, int D1, typename T, int NG>
__device__ __forceinline__ T pick(const T (&v)[NG], unsigned m0) {
  static_assert(D0 < NG && D1 < NG, "group within the loaded parameters");
  if constexpr (D0 == D1) {
    return v[D0];
  } else {
    unsigned a, b;
    __builtin_memcpy(&a, &v[D0], 4);
    __builtin_memcpy(&b, &v[D1], 4);
    const unsigned r = (m0 & a) | (~m0 & b);
    T t;
    __builtin_memcpy(&t, &r, 4);
    return t;
  }
}
// group of code e of slot S in phase PH for lane half h (qp_dg)
#define QP_DG(h, e) qp_dg(KQ, GS, PH, h, S, e)

// INT4 chunk of slot S (phase PH) -> 8 fp16 weights; code e uses its own
// group's parameters.
template <int KQ, int GS, int PH, int S, int NG>
__device__ __forceinline__ uint4 dq_int4(unsigned w, const DqGroups<NG>& p, unsigned m0, const DqConsts<Q_INT4>& k) {
  const unsigned w8 = w >> 8;
  const unsigned u0 = (w & k.m_lo) | k.c1024;   // e0, e1: 1024 + q
  const unsigned u1 = (w & k.m_hi) | k.c64;     // e2, e3: 64 + q
  const unsigned u2 = (w8 & k.m_lo) | k.c1024;  // e4, e5
  const unsigned u3 = (w8 & k.m_hi) | k.c64;    // e6, e7
#define QP_S(e) pick<QP_DG(0, e), QP_DG(1, e)>(p.s, m0)
#define QP_B(e, off) pick<QP_DG(0, e), QP_DG(1, e)>(p.off, m0)
  return make_uint4(fmix2(u0, QP_S(0), QP_B(0, b1024), QP_S(1), QP_B(1, b1024)),
                    fmix2(u1, QP_S(2), QP_B(2, b64), QP_S(3), QP_B(3, b64)),
                    fmix2(u2, QP_S(4), QP_B(4, b1024), QP_S(5), QP_B(5, b1024)),
                    fmix2(u3, QP_S(6), QP_B(6, b64), QP_S(7), QP_B(7, b64)));
}

template <int KQ, int GS, int PH, int S, int NG>
__device__ __forceinline__ uint4 dq_int8(unsigned w0, unsigned w1, const DqGroups<NG>& p, unsigned m0,
                                         const DqConsts<Q_INT8>& k) {
  // v_perm_b32: selector bytes 0..3 pick bytes of the second operand (the codes),
  // 4..7 bytes of the first (0x64): (q_e, 0x64, q_e+1, 0x64) = fp16 1024 + q
  const unsigned u0 = __builtin_amdgcn_perm(k.c64x4, w0, 0x04010400u);
  const unsigned u1 = __builtin_amdgcn_perm(k.c64x4, w0, 0x04030402u);
  const unsigned u2 = __builtin_amdgcn_perm(k.c64x4, w1, 0x04010400u);
  const unsigned u3 = __builtin_amdgcn_perm(k.c64x4, w1, 0x04030402u);
  return make_uint4(fmix2(u0, QP_S(0), QP_B(0, b1024), QP_S(1), QP_B(1, b1024)),
                    fmix2(u1, QP_S(2), QP_B(2, b1024), QP_S(3), QP_B(3, b1024)),
                    fmix2(u2, QP_S(4), QP_B(4, b1024), QP_S(5), QP_B(5, b1024)),
                    fmix2(u3, QP_S(6), QP_B(6, b1024), QP_S(7), QP_B(7, b1024)));
#undef QP_B
#undef QP_S
}

// fp16 scale pair of codes (e, e + 1): both halves from one group when the two
// codes share it (the usual case), else the low half of e's and the high half
// of e + 1's.
template <int KQ, int GS, int PH, int S, int E, int NG>
__device__ __forceinline__ unsigned tern_scales(const DqGroups<NG>& p, unsigned m0) {
  const unsigned lo = pick<QP_DG(0, E), QP_DG(1, E)>(p.h, m0);
  if constexpr (QP_DG(0, E) == QP_DG(0, E + 1) && QP_DG(1, E) == QP_DG(1, E + 1)) return lo;
  else return (lo & 0x0000FFFFu) | (pick<QP_DG(0, E + 1), QP_DG(1, E + 1)>(p.h, m0) & 0xFFFF0000u);
}

// Ternary chunk of slot S (phase PH) in layout A (LB = 0: code 2p at bit 2p,
// 2p+1 at 16+2p) or B (LB = 1: bits 8+2p, 24+2p) -> 8 fp16 weights t * fp16(s).
// v_perm_b32 picks each value's high byte from {0xBC, 0x00, 0x3C, 0x00}
// (code 0 -> -1.0, 1 -> 0, 2 -> +1.0, 3 -> 0); selector 12 yields the zero low
// bytes.  Each code is scaled by its own group's scale.
template <int KQ, int GS, int PH, int S, int LB, int NG>
__device__ __forceinline__ uint4 dq_tern(unsigned w, const DqGroups<NG>& p, unsigned m0, const DqConsts<Q_TERN>& k) {
  constexpr unsigned kTable = 0x003C00BCu;
  unsigned o[4];
  static_for<0, 4>([&](auto QC) __attribute__((always_inline)) {
    constexpr int q = decltype(QC)::value;
    const unsigned v = LB ? (w >> (2 * q)) : (w << (8 - 2 * q));
    const unsigned sel = (v & k.t_mask) | k.t_zero;
    const unsigned t = __builtin_amdgcn_perm(0u, kTable, sel);
    const unsigned sc = tern_scales<KQ, GS, PH, S, 2 * q, NG>(p, m0);
    half2_t th, sh;
    __builtin_memcpy(&th, &t, 4);
    __builtin_memcpy(&sh, &sc, 4);
    const half2_t r = th * sh;
    __builtin_memcpy(&o[q], &r, 4);
  });
  return make_uint4(o[0], o[1], o[2], o[3]);
}
#undef QP_DG

// 16-bit ternary chunk (code 2p at bit 2p, 2p+1 at bit 8+2p) -> layout A
__device__ __forceinline__ unsigned tern_spread(unsigned h) { return (h & 0xFFu) | ((h & 0xFF00u) << 8); }

// Loads of N bytes at p (N in {2, 4, 8, 16, 32}) into dwords (2 bytes: the low half).
template <int N>
__device__ __forceinline__ void load_bytes(const unsigned char* p, unsigned* out) {
  if constexpr (N == 2) {
    out[0] = *reinterpret_cast<const unsigned short*>(p);
  } else if constexpr (N == 4) {
    out[0] = *reinterpret_cast<const unsigned*>(p);
  } else if constexpr (N == 8) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    out[0] = v.x;
    out[1] = v.y;
  } else {
    static_assert(N % 16 == 0, "chunk records of 2, 4, 8 or 16k bytes");
#pragma unroll
    for (int i = 0; i < N / 16; ++i) {
      const uint4 v = reinterpret_cast<const uint4*>(p)[i];
      out[4 * i + 0] = v.x;
      out[4 * i + 1] = v.y;
      out[4 * i + 2] = v.z;
      out[4 * i + 3] = v.w;
    }
  }
}

__device__ __forceinline__ float load_any_f(const void* p, long i, int dt) {
  if (dt == DT_F32) return reinterpret_cast<const float*>(p)[i];
  if (dt == DT_F16) return (float)reinterpret_cast<const _Float16*>(p)[i];
  return to_f32(reinterpret_cast<const __bf16*>(p)[i]);
}

// SiLU with the +-20 clip of the exponent argument (gated_kan.py:15-16).
__device__ __forceinline__ float silu_clip20(float g) {
  const float c = fminf(fmaxf(g, -20.0f), 20.0f);
  return g / (1.0f + __expf(-c));
}
__device__ __forceinline__ float round16v(float v, int mode) {
  asm volatile("" : "+v"(v));
  return mode == 2 ? to_f32(from_f32<__bf16>(v)) : mode == 1 ? (float)(_Float16)v : v;
}

__device__ __forceinline__ void store_any(void* Y, long i, int dt, float v) {
  if (dt == DT_F32) reinterpret_cast<float*>(Y)[i] = v;
  else if (dt == DT_F16) reinterpret_cast<_Float16*>(Y)[i] = (_Float16)v;
  else reinterpret_cast<__bf16*>(Y)[i] = (__bf16)v;
}

// emit<KN> of the B-spline table generator into the A fragments a
template <int KN, typename G, typename Frag>
__device__ __forceinline__ void gen_emit_tab(const G& g, Frag (&a)[1]) {
  g.template emit<KN>(a);
}

struct QPArgs {
  const void* X;
  long ldx;
  int x_f32;
  QPMat m[2];
  int grp;
  int bias_dt;
  void* Y;
  long ldy;
  int y_dt;
  float* part;
  int B, D_in, m_tiles, n_tiles, nfb, fb_per_split;
  int epi, round16;
  BasisParams bp;  // RBF / B-spline parameters
  int pair;        // dispatch: two feature blocks per LDS stage (PAIR instantiation) where built
};

}  // namespace

// ---------------------------------------------------------------------------
// The fused kernel.  QT: Q_INT4 / Q_INT8 / Q_TERN; KQ: basis functions per
// feature (1 .. kQPMaxK); HB: SiLU base branch; BASIS: the A-fragment generator
// (BASIS_CHEBY_POST, BASIS_RBF_REC, BASIS_BSPLINE; see BasisGen).  Grid:
// m_tiles * n_tiles workgroups (x) by feature splits (y), 512 threads.
// PAIR: each LDS stage holds two feature blocks (2 KP <= 10 slots, a group
// geometry that repeats every block): one barrier per two blocks, and the
// block decoded during block fb is fb + 2, into the same half of the other
// stage.  The arithmetic and its order are those of one block per stage.
// ---------------------------------------------------------------------------
template <int QT, int KQ, int HB, int BASIS = BASIS_CHEBY_POST, bool PAIR = false>
__global__ void __launch_bounds__(kQThreads, 1) kan_qfused_block(QPArgs A) {
  constexpr int KP = KQ + HB;
  constexpr int NV = 8;
  constexpr int SLOT = kQNB * 64;  // uint4 per slot of the N-tile
  constexpr int CB = qp_chunk_bytes(QT);
  constexpr int GS = qp_group(QT);
  constexpr int PF = qp_param_floats(QT);
  // basis code dwords per block (ternary: one per slot pair, an odd K padded)
  constexpr int NCB = QT == Q_TERN ? (KQ == 1 ? 1 : (KQ + 1) / 2) : (KQ * CB) / 4;
  constexpr int NCW = QT == Q_INT8 ? 2 : 1;  // base code dwords
  typedef half8 frag;
  static_assert(KQ >= 1 && KQ <= kQPMaxK && KP <= 10, "K + base slots of fp16 B-tiles in two LDS stages");
  // quantization groups a half-block's codes meet, and the phases of the
  // feature block index that place them differently (qp_ngroups, qp_period)
  constexpr int NGRP = qp_ngroups(KQ, GS);
  constexpr int PER = qp_period(KQ, GS);
  static_assert(NGRP <= 3 && (PER == 1 || PER == 2 || PER == 4), "group geometry");

  static_assert(!PAIR || (PER == 1 && 2 * KP <= 10 && BASIS != BASIS_BSPLINE_TAB), "block pairs");
  constexpr int AH = PAIR ? 2 : 1;          // blocks between the one multiplied and the one decoded
  constexpr int HALF = KP * SLOT;           // uint4 of one feature block's tiles
  __shared__ uint4 stage0[(PAIR ? 2 : 1) * HALF];
  __shared__ uint4 stage1[(PAIR ? 2 : 1) * HALF];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int m_tile, n_tile;
  tile_of(xcd_remap(blockIdx.x, A.m_tiles * A.n_tiles), A.m_tiles, A.n_tiles, m_tile, n_tile);
  const int split = blockIdx.y;
  const int row0 = m_tile * (kQWaves * 32) + wave * 32;
  const int fb_begin = split * A.fb_per_split;
  const int fb_end = min(A.nfb, fb_begin + A.fb_per_split);
  if (fb_end <= fb_begin) return;  // uniform per workgroup (empty split)
  const int B = A.B, D_in = A.D_in;

  // ---- this wave's decode role: column block `wave` of the N-tile ----------
  const int mi = A.grp == 4 ? (wave >> 2) : 0;
  const QPMat M = mi ? A.m[1] : A.m[0];
  const int ob = n_tile * A.grp + (wave & (A.grp - 1));
  const int hh = lane >> 5;
  const int o = ob * 32 + (lane & 31);
  const long rec = (long)ob * 64 + lane;  // chunk record of (fb = 0, ob, lane)
  const long fb_stride = (long)M.nob_pad * 64;
  DqConsts<QT> dk;
  dk.init();

  // One register set holds the codes and parameters of the next feature block
  // to decode; each slot's chunk word is refilled with the following block's
  // as soon as it has been decoded (load-to-use distance: one block).
  struct QRegs {
    unsigned cb[NCB];
    unsigned cw[NCW];
    float pb[NGRP * PF], pw[PF];
  };
  // chunk words of segment / slot group g of feature block fbq (clamped into
  // the split: loads past it re-read the last block, in bounds).  Codes are
  // laid out [fb][ob][g][lane], one 64-lane word group per slot (ternary with
  // K > 1: per slot pair), so each load is one coalesced 64-lane access.
  constexpr int WB = QT == Q_TERN ? (KQ == 1 ? 2 : 4) : CB;                 // bytes of one basis word group entry
  constexpr int NG = QT == Q_TERN ? (KQ == 1 ? 1 : (KQ + 1) / 2) : KQ;  // basis word groups per block
  // Every address is a wave-uniform base (feature block, column block, slot
  // group) plus this lane's fixed byte offset, so the loads take the
  // scalar-base + 32-bit vector-offset form and cost no per-block VALU.
  // The first group of a lane's half-block is floor(16 f K / GS) (uniform)
  // plus qp_gl(f mod PER, hh) (a lane constant per phase); the base segment
  // (K = 1) never leaves group floor(16 f / GS).
  const bool hi = hh != 0;
  unsigned m0 = hi ? 0u : ~0u;  // lane-half mask of the per-code group selects (pick)
  asm volatile("" : "+v"(m0));
  const unsigned cb_off = (unsigned)lane * WB, cw_off = (unsigned)lane * CB;
  unsigned pb_off[PER];
  static_for<0, PER>([&](auto PHC) __attribute__((always_inline)) {
    constexpr int ph = decltype(PHC)::value;
    constexpr int gl0 = qp_gl(KQ, GS, ph, 0), gl1 = qp_gl(KQ, GS, ph, 1);
    pb_off[ph] = (unsigned)(((hi ? gl1 : gl0) * M.ldp + o) * PF * 4);
  });
  const unsigned pw_off = (unsigned)(o * PF * 4);
  auto load_cb = [&](int fbq, int g, QRegs& r) __attribute__((always_inline)) {
    const int f = min(fbq, fb_end - 1);
    const unsigned char* ub = M.cb + (((long)f * M.nob_pad + ob) * NG + g) * (64 * WB);
    load_bytes<WB>(ub + cb_off, &r.cb[g * (WB >= 4 ? WB / 4 : 1)]);
  };
  auto load_cw = [&](int fbq, QRegs& r) __attribute__((always_inline)) {
    const int f = min(fbq, fb_end - 1);
    load_bytes<CB>(M.cw + ((long)f * M.nob_pad + ob) * (64 * CB) + cw_off, r.cw);
  };
  // parameters of block fbq, whose phase (fbq mod PER) is PHC; a block past the
  // split is clamped to its last one (its parameters are never used, and the
  // zero rows past the last group keep the loads in bounds)
  auto load_params = [&](int fbq, auto PHC, QRegs& r) __attribute__((always_inline)) {
    constexpr int ph = decltype(PHC)::value;
    const int f = min(fbq, fb_end - 1);
    const char* pb = reinterpret_cast<const char*>(M.pb + (long)((16 * f * KQ) / GS) * M.ldp * PF) + pb_off[ph];
#pragma unroll
    for (int d = 0; d < NGRP; ++d) {
      const float* pd = reinterpret_cast<const float*>(pb + (long)d * M.ldp * PF * 4);
      r.pb[d * PF] = pd[0];
      if constexpr (PF == 2) r.pb[d * PF + 1] = pd[1];
    }
    if constexpr (HB) {
      const char* pw = reinterpret_cast<const char*>(M.pw + (long)((16 * f) / GS) * M.ldp * PF) + pw_off;
      r.pw[0] = reinterpret_cast<const float*>(pw)[0];
      if constexpr (PF == 2) r.pw[1] = reinterpret_cast<const float*>(pw)[1];
    }
  };
  auto load_all = [&](int fbq, auto PHC, QRegs& r) __attribute__((always_inline)) {
    static_for<0, NG>([&](auto G) __attribute__((always_inline)) { load_cb(fbq, decltype(G)::value, r); });
    if constexpr (HB) load_cw(fbq, r);
    load_params(fbq, PHC, r);
  };
  // after slot SC's chunk has been decoded: refill its word (group) for block fbq
  auto reload_slot = [&](auto SCC, int fbq, QRegs& r) __attribute__((always_inline)) {
    constexpr int SC = decltype(SCC)::value;
    if constexpr (HB && SC == 0) {
      load_cw(fbq, r);
    } else {
      constexpr int k = SC - HB;
      if constexpr (QT != Q_TERN || KQ == 1) load_cb(fbq, k, r);
      else if constexpr ((k & 1) || k == KQ - 1) load_cb(fbq, k / 2, r);  // every slot of the word decoded
    }
  };
  // decoded chunk of slot SC (compile time) of a block in phase PHC, from the
  // registers of that block
  auto dq_slot = [&](auto SCC, auto PHC, const QRegs& r, const DqGroups<NGRP>& pb, const DqGroups<1>& pw)
      __attribute__((always_inline)) -> uint4 {
    constexpr int SC = decltype(SCC)::value;
    constexpr int ph = decltype(PHC)::value;
    if constexpr (HB && SC == 0) {
      // base segment: K = 1, one group per half-block
      if constexpr (QT == Q_INT4) return dq_int4<1, GS, 0, 0>(r.cw[0], pw, m0, dk);
      else if constexpr (QT == Q_INT8) return dq_int8<1, GS, 0, 0>(r.cw[0], r.cw[1], pw, m0, dk);
      else return dq_tern<1, GS, 0, 0, 0>(tern_spread(r.cw[0]), pw, m0, dk);
    } else {
      constexpr int k = SC - HB;
      if constexpr (QT == Q_INT4) return dq_int4<KQ, GS, ph, k>(r.cb[k], pb, m0, dk);
      else if constexpr (QT == Q_INT8) return dq_int8<KQ, GS, ph, k>(r.cb[2 * k], r.cb[2 * k + 1], pb, m0, dk);
      else if constexpr (KQ == 1) return dq_tern<KQ, GS, ph, k, 0>(tern_spread(r.cb[0]), pb, m0, dk);
      else return dq_tern<KQ, GS, ph, k, k & 1>(r.cb[k / 2], pb, m0, dk);
    }
  };
  auto params_of = [&](const QRegs& r, DqGroups<NGRP>& pb, DqGroups<1>& pw) __attribute__((always_inline)) {
#pragma unroll
    for (int d = 0; d < NGRP; ++d) {
      if constexpr (QT == Q_TERN) {
        pb.h[d] = half2_of(r.pb[d]);
      } else {
        pb.s[d] = r.pb[2 * d];
        pb.b1024[d] = __builtin_fmaf(-1024.0f, r.pb[2 * d], r.pb[2 * d + 1]);
        pb.b64[d] = __builtin_fmaf(-64.0f, r.pb[2 * d], r.pb[2 * d + 1]);
      }
    }
    if constexpr (HB) {
      if constexpr (QT == Q_TERN) {
        pw.h[0] = half2_of(r.pw[0]);
      } else {
        pw.s[0] = r.pw[0];
        pw.b1024[0] = __builtin_fmaf(-1024.0f, r.pw[0], r.pw[1]);
        pw.b64[0] = __builtin_fmaf(-64.0f, r.pw[0], r.pw[1]);
      }
    }
  };
  // Features 16 fbq + 8 (lane / 32) + e at or past D_in must contribute zero
  // weights (their affine group parameters belong to real features too): in
  // the last feature block of a ragged D_in (a wave-uniform condition) the
  // decoded halves of those features are cleared.
  auto is_tail = [&](int fbq) __attribute__((always_inline)) -> bool { return 16 * (min(fbq, fb_end - 1) + 1) > D_in; };
  auto mask_tail = [&](int fbq, uint4& v) __attribute__((always_inline)) {
    const int nv = max(0, min(8, D_in - (16 * min(fbq, fb_end - 1) + 8 * hh)));
    v.x &= (0 < nv ? 0x0000FFFFu : 0u) | (1 < nv ? 0xFFFF0000u : 0u);
    v.y &= (2 < nv ? 0x0000FFFFu : 0u) | (3 < nv ? 0xFFFF0000u : 0u);
    v.z &= (4 < nv ? 0x0000FFFFu : 0u) | (5 < nv ? 0xFFFF0000u : 0u);
    v.w &= (6 < nv ? 0x0000FFFFu : 0u) | (7 < nv ? 0xFFFF0000u : 0u);
  };

  // ---- inputs (as kan_fused_block): lane holds x[row0 + lane%32][16 fb + 8 (lane/32) + j]
  uint4 xr[2];
  auto xload = [&](int fbx) __attribute__((always_inline)) {
    const int f0 = fbx * 16 + 8 * hh;
    const int row = row0 + (lane & 31);
    const bool ok = (row < B) && (f0 < D_in);
    if (A.x_f32) {
      const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(A.X) + (long)row * A.ldx + f0);
      xr[0] = ok ? p[0] : make_uint4(0, 0, 0, 0);
      xr[1] = ok ? p[1] : make_uint4(0, 0, 0, 0);
    } else {
      const uint4* p =
          reinterpret_cast<const uint4*>(reinterpret_cast<const _Float16*>(A.X) + (long)row * A.ldx + f0);
      xr[0] = ok ? p[0] : make_uint4(0, 0, 0, 0);
    }
  };
  auto xunpack = [&](int fbx, float* xf) __attribute__((always_inline)) {
    const int f0 = fbx * 16 + 8 * hh;
    if (A.x_f32) {
      const unsigned w[8] = {xr[0].x, xr[0].y, xr[0].z, xr[0].w, xr[1].x, xr[1].y, xr[1].z, xr[1].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) xf[j] = __uint_as_float(w[j]);
    } else {
      const unsigned w[4] = {xr[0].x, xr[0].y, xr[0].z, xr[0].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        half2_t h;
        __builtin_memcpy(&h, &w[q], 4);
        xf[2 * q] = (float)h[0];
        xf[2 * q + 1] = (float)h[1];
      }
    }
    if ((fbx + 1) * 16 > D_in) {
#pragma unroll
      for (int j = 0; j < NV; ++j)
        if (f0 + j >= D_in) xf[j] = 0.0f;
    }
  };
  auto pack = [&](frag& a, const float* v) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = (_Float16)v[j];
  };
  auto bread = [&](frag (&b)[kQNB], const uint4* stage, int s) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < kQNB; ++nb) {
      uint4 u = stage[(s * kQNB + nb) * 64 + lane];
      b[nb] = *reinterpret_cast<frag*>(&u);
    }
  };

  floatx16 acc[kQNB];
#pragma unroll
  for (int nb = 0; nb < kQNB; ++nb)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[nb][r] = 0.0f;

  __shared__ uint4 bs_sel[kBsplineTabG];  // B-spline table: perm selectors per span (kTab)
  if constexpr (BASIS == BASIS_BSPLINE_TAB) {
    if (tid < kBsplineTabG)
      bs_sel[tid] = make_uint4(bspline_tab_selector(tid, 0), bspline_tab_selector(tid, 1),
                               bspline_tab_selector(tid, 2), bspline_tab_selector(tid, 3));
  }

  // ---- prologue: block fb_begin decoded into stage0, fb_begin + 1 in registers
  QRegs R;
  // fb_begin is a multiple of PER (the host rounds the split size): phase 0
  using Ph0 = std::integral_constant<int, 0>;
  using Ph1 = std::integral_constant<int, 1 % PER>;
  load_all(fb_begin, Ph0{}, R);
  xload(fb_begin);
  {
    DqGroups<NGRP> pb;
    DqGroups<1> pw;
    params_of(R, pb, pw);
    const bool tail = is_tail(fb_begin);
    // each slot straight to LDS (an array of the decoded slots was placed in
    // memory at the larger K)
    static_for<0, KP>([&](auto SCC) __attribute__((always_inline)) {
      constexpr int SC = decltype(SCC)::value;
      uint4 d = dq_slot(SCC, Ph0{}, R, pb, pw);
      if (tail) mask_tail(fb_begin, d);
      stage0[(SC * kQNB + wave) * 64 + lane] = d;
    });
    load_all(fb_begin + 1, Ph1{}, R);
  }
  if constexpr (PAIR) {
    // block fb_begin + 1 into the second half of stage 0 (past the split: the
    // clamped last block, never read); the registers then hold fb_begin + 2
    DqGroups<NGRP> pb;
    DqGroups<1> pw;
    params_of(R, pb, pw);
    const bool tail = is_tail(fb_begin + 1);
    static_for<0, KP>([&](auto SCC) __attribute__((always_inline)) {
      constexpr int SC = decltype(SCC)::value;
      uint4 d = dq_slot(SCC, Ph0{}, R, pb, pw);
      if (tail) mask_tail(fb_begin + 1, d);
      stage0[HALF + (SC * kQNB + wave) * 64 + lane] = d;
    });
    load_all(fb_begin + 2, Ph0{}, R);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes are done
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // B-spline with G = 5 (K = 8): the per-input table of BsplineTab (one v_perm_b32 per two values and
  // slot; its 5 selector rows in LDS, written before the prologue's barrier)
  constexpr bool kTab = BASIS == BASIS_BSPLINE_TAB;
  static_assert(!kTab || KQ == kBsplineTabG + 3, "B-spline table: G = 5");
  typedef typename std::conditional<kTab, BsplineTab<_Float16, NV>, BasisGen<kTab ? BASIS_CHEBY_POST : BASIS, NV>>::type Gen;
  Gen gen;
  const BasisParams& bp = A.bp;
  frag af[2], bf[kQNB];
  // emit basis KN of the table generator into A fragment a
  auto tab_emit = [&](auto KNC, frag& a) __attribute__((always_inline)) {
    frag(&a1)[1] = *reinterpret_cast<frag(*)[1]>(&a);
    gen_emit_tab<decltype(KNC)::value>(gen, a1);
  };

  // One feature block: MFMAs of block fb from `cur`, decode of block fb + AH
  // (in R) into `nxt`, R refilled with block fb + AH + 1.
  // PHC: the phase of fb (fb mod PER); block fb + 1 is decoded in the next
  // phase, and R is refilled with block fb + 2 in the one after (PAIR: one
  // phase, PER = 1).  SYNC: end with the barrier (PAIR: every second block).
  auto block = [&](int fb, const uint4* cur, uint4* nxt, auto PHC, auto SYNC) __attribute__((always_inline)) {
    constexpr int ph = decltype(PHC)::value;
    using PhN = std::integral_constant<int, (ph + 1) % PER>;
    using PhNN = std::integral_constant<int, (ph + 2) % PER>;
    float xf[NV];
    xunpack(fb, xf);
    if (fb + 1 < fb_end) xload(fb + 1);
    DqGroups<NGRP> pb;
    DqGroups<1> pw;
    params_of(R, pb, pw);
    const bool tail = is_tail(fb + AH);
    load_params(fb + AH + 1, PhNN{}, R);
    bread(bf, cur, 0);
    if constexpr (kTab) gen.begin(xf, bp, bs_sel);
    else gen.begin(xf, bp, HB != 0);
    {
      float v[NV];
      if constexpr (HB) {
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = silu_f32(xf[i]);
        pack(af[0], v);
      } else if constexpr (kTab) {
        tab_emit(std::integral_constant<int, 0>{}, af[0]);
      } else {
        gen.template step<0>(0, bp, v);
        pack(af[0], v);
      }
    }
    // slot 0's B-fragment reads stay ahead of the slots' scheduling regions:
    // inside slot 0's the scheduler placed each just before its MFMA, which
    // then waited for it
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, KP>([&](auto SCC) __attribute__((always_inline)) {
      constexpr int SC = decltype(SCC)::value;
      constexpr int P = SC & 1;
      // basis values of slot SC + 1 (basis function SC + 1 - HB) into the other A fragment
      if constexpr (SC + 1 < KP) {
        if constexpr (kTab) {
          tab_emit(std::integral_constant<int, SC + 1 - HB>{}, af[P ^ 1]);
        } else {
          float v[NV];
          gen.template step<P ^ 1>(SC + 1 - HB, bp, v);
          pack(af[P ^ 1], v);
        }
      }
      // decode slot SC of block fb + AH, then refill its code word with block fb + AH + 1
      const uint4 d = dq_slot(SCC, PhN{}, R, pb, pw);
      reload_slot(SCC, fb + AH + 1, R);
#pragma unroll
      for (int nb = 0; nb < kQNB; ++nb) {
        acc[nb] = Mfma<_Float16>::mma(af[P], bf[nb], acc[nb]);
        if constexpr (SC + 1 < KP) {
          uint4 u = cur[((SC + 1) * kQNB + nb) * 64 + lane];
          bf[nb] = *reinterpret_cast<frag*>(&u);
        }
      }
      nxt[(SC * kQNB + wave) * 64 + lane] = d;
      // issue order: per column block one MFMA, a share of the VALU work (up to
      // 8 instructions: a slot has ~60, so all of them sit between MFMAs; 4 left
      // some after the last MFMA, 0.8 % slower for INT4 / INT8, 6 was slower,
      // 10 no faster), the next slot's B-fragment read; the decoded chunk's LDS
      // write last
#pragma unroll
      for (int nb = 0; nb < kQNB; ++nb) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // VALU
        if constexpr (SC + 1 < KP) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      }
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
      __builtin_amdgcn_sched_barrier(0);
    });
    // a ragged last feature block: clear the padded features' weights of this
    // wave's chunks (LDS operations of a wave complete in order), outside the
    // slots' basic blocks
    if (tail) {
#pragma unroll
      for (int sc = 0; sc < KP; ++sc) {
        uint4 v = nxt[(sc * kQNB + wave) * 64 + lane];
        mask_tail(fb + AH, v);
        nxt[(sc * kQNB + wave) * 64 + lane] = v;
      }
    }
    // the decoded block is in LDS (lgkmcnt(0)) and every wave is done with `cur`;
    // the register loads stay in flight across the barrier
    if constexpr (decltype(SYNC)::value) {
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
  };
  using Sync = std::true_type;
  using NoSync = std::false_type;
  if constexpr (PAIR) {
    // stage s holds blocks fb (first half) and fb + 1 (second half); the closing
    // barrier runs on every path (the conditions are uniform per workgroup)
    auto barrier = [&]() __attribute__((always_inline)) {
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    for (int fb = fb_begin; fb < fb_end; fb += 4) {
      block(fb, stage0, stage1, Ph0{}, NoSync{});
      if (fb + 1 < fb_end) block(fb + 1, stage0 + HALF, stage1 + HALF, Ph0{}, NoSync{});
      barrier();
      if (fb + 2 < fb_end) {
        block(fb + 2, stage1, stage0, Ph0{}, NoSync{});
        if (fb + 3 < fb_end) block(fb + 3, stage1 + HALF, stage0 + HALF, Ph0{}, NoSync{});
        barrier();
      }
    }
  } else {
    constexpr int UNR = PER == 4 ? 4 : 2;  // blocks per loop round: the stages alternate, phases repeat
    for (int fb = fb_begin; fb < fb_end; fb += UNR) {
      block(fb, stage0, stage1, Ph0{}, Sync{});
      if (fb + 1 < fb_end) block(fb + 1, stage1, stage0, Ph1{}, Sync{});
      if constexpr (PER == 4) {
        if (fb + 2 < fb_end) block(fb + 2, stage0, stage1, std::integral_constant<int, 2>{}, Sync{});
        if (fb + 3 < fb_end) block(fb + 3, stage1, stage0, std::integral_constant<int, 3>{}, Sync{});
      }
    }
  }

  // ---- epilogue -------------------------------------------------------------
  // acc register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l%32.
  const int rbase = row0 + 4 * (lane >> 5);
  if (A.part != nullptr) {
    const long ncols = (long)A.n_tiles * 256;
#pragma unroll
    for (int nb = 0; nb < kQNB; ++nb) {
      const long col = (long)n_tile * 256 + nb * 32 + (lane & 31);
      float* out = A.part + ((long)split * B + rbase) * ncols + col;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dr = 8 * (r >> 2) + (r & 3);
        if (rbase + dr < B) out[(long)dr * ncols] = acc[nb][r];
      }
    }
    return;
  }
  if (A.epi == QP_EPI_SWIGLU) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int c = (n_tile * 4 + nb) * 32 + (lane & 31);
      if (c < A.m[0].D_out) {
        const float bg = A.m[0].bias ? load_any_f(A.m[0].bias, c, A.bias_dt) : 0.0f;
        const float bu = A.m[1].bias ? load_any_f(A.m[1].bias, c, A.bias_dt) : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dr = 8 * (r >> 2) + (r & 3);
          if (rbase + dr < B) {
            const float g = round16v(acc[nb][r] + bg, A.round16);
            const float u = round16v(acc[nb + 4][r] + bu, A.round16);
            const float h = round16v(silu_clip20(g) * u, A.round16);
            store_any(A.Y, (long)(rbase + dr) * A.ldy + c, A.y_dt, h);
          }
        }
      }
    }
    return;
  }
#pragma unroll
  for (int nb = 0; nb < kQNB; ++nb) {
    const int c = (n_tile * 8 + nb) * 32 + (lane & 31);
    if (c < A.m[0].D_out) {
      const float bc = A.m[0].bias ? load_any_f(A.m[0].bias, c, A.bias_dt) : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dr = 8 * (r >> 2) + (r & 3);
        if (rbase + dr < B) store_any(A.Y, (long)(rbase + dr) * A.ldy + c, A.y_dt, acc[nb][r] + bc);
      }
    }
  }
}

template <int QT, int KQ, int HB, int BASIS>
static void qp_go(const QPArgs& A, dim3 grid, hipStream_t st) {
  // two feature blocks per stage: Chebyshev K = 4 (the GatedKAN shape; its groups repeat every block)
  if constexpr (BASIS == BASIS_CHEBY_POST && KQ == 4) {
    if (A.pair) {
      hipLaunchKernelGGL((kan_qfused_block<QT, KQ, HB, BASIS, true>), grid, dim3(kQThreads), 0, st, A);
      return;
    }
  }
  hipLaunchKernelGGL((kan_qfused_block<QT, KQ, HB, BASIS>), grid, dim3(kQThreads), 0, st, A);
}

// Instantiated (QT, K, basis) combinations: qp_supported.
template <int QT, int HB, int BASIS>
static hipError_t qp_dispatch_k(const QPLaunch& L, const QPArgs& A, dim3 grid, hipStream_t st) {
#define QP_K(KV)                                                   \
  if (L.K == KV) {                                                 \
    qp_go<QT, KV, HB, BASIS>(A, grid, st);                         \
    return hipGetLastError();                                      \
  }
  if constexpr (BASIS == BASIS_BSPLINE_TAB) {
    if constexpr (QT != Q_INT8) QP_K(8)
  } else if constexpr (BASIS == BASIS_BSPLINE) {
    QP_K(4)
  } else {
    if constexpr (BASIS == BASIS_CHEBY_POST) QP_K(1)
    QP_K(2)
    QP_K(3)
    QP_K(4)
    QP_K(5)
    QP_K(6)
    if constexpr (!(QT == Q_INT8 && HB)) QP_K(7)
    QP_K(8)
    QP_K(9)
  }
#undef QP_K
  return hipErrorInvalidValue;
}

template <int QT, int HB>
static hipError_t qp_dispatch_basis(const QPLaunch& L, const QPArgs& A, dim3 grid, hipStream_t st) {
  switch (L.basis) {
    case BASIS_CHEBY: return qp_dispatch_k<QT, HB, BASIS_CHEBY_POST>(L, A, grid, st);
    case BASIS_RBF: return qp_dispatch_k<QT, HB, BASIS_RBF_REC>(L, A, grid, st);
    default:  // G = 5 (K = 8): the basis table; other G: per-value selection
      if (L.K == kBsplineTabG + 3) return qp_dispatch_k<QT, HB, BASIS_BSPLINE_TAB>(L, A, grid, st);
      return qp_dispatch_k<QT, HB, BASIS_BSPLINE>(L, A, grid, st);
  }
}

// One fused launch of format QT (base branch HB) on the grid the host launcher chose.
template <int QT, int HB>
hipError_t qp_run(const QPLaunch& L, const QPGrid& G, hipStream_t st) {
  QPArgs A{};
  A.X = L.X;
  A.ldx = L.ldx;
  A.x_f32 = L.x_dtype == DT_F32;
  A.m[0] = L.m[0];
  A.m[1] = L.grp == 4 ? L.m[1] : L.m[0];
  A.grp = L.grp;
  A.bias_dt = L.bias_dtype;
  A.Y = L.Y;
  A.ldy = L.ldy;
  A.y_dt = L.y_dtype;
  A.B = L.B;
  A.D_in = L.D_in;
  A.m_tiles = G.m_tiles;
  A.n_tiles = G.n_tiles;
  A.nfb = G.nfb;
  A.fb_per_split = G.fb_per_split;
  A.part = G.nsp > 1 ? L.part : nullptr;
  A.epi = L.epi;
  A.round16 = L.round16;
  A.bp = L.bp;
  A.pair = g_qp_block_pairs;
  return qp_dispatch_basis<QT, HB>(L, A, dim3((unsigned)(G.m_tiles * G.n_tiles), (unsigned)G.nsp), st);
}

}  // namespace kans
