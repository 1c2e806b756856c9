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

// fp16 pair (V0, V1) -> (fp16(V0*s + off), fp16(V1*s + off)), each one fma in
// fp32 with an fp16 source and an fp16 result: v_fma_mixlo_f16 writes the low
// half, v_fma_mixhi_f16 the high half of the same register (the compiler
// builds the pair from two mixlo results, a shift and an or instead).
// op_sel_hi:[1,0,0] reads src0 as fp16 (op_sel picks its half), s and off as
// fp32.
__device__ __forceinline__ unsigned fmix2(unsigned u, float s, float off) {
  unsigned r;
  asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(u), "v"(s), "v"(off));
  asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(r) : "v"(u), "v"(s), "v"(off));
  return r;
}

// Per-segment decode parameters of one chunk (set once per feature block).
struct DqParams {
  float s, b1024, b64;  // affine: scale, bias - 1024 s, bias - 64 s
  unsigned s16x2;       // ternary: fp16(scale) in both halves
  unsigned s16x2b;      // ternary at K = 8: fp16(scale) of codes 4-7 (the next group)
};

__device__ __forceinline__ DqParams dq_params_affine(float s, float b) {
  DqParams p;
  p.s = s;
  p.b1024 = __builtin_fmaf(-1024.0f, s, b);
  p.b64 = __builtin_fmaf(-64.0f, s, b);
  p.s16x2 = p.s16x2b = 0u;
  return p;
}
__device__ __forceinline__ unsigned half2_of(float s) {
  const _Float16 h = (_Float16)s;
  unsigned short u;
  __builtin_memcpy(&u, &h, 2);
  return (unsigned)u | ((unsigned)u << 16);
}
__device__ __forceinline__ DqParams dq_params_tern(float s, float s_b) {
  DqParams p;
  p.s = p.b1024 = p.b64 = 0.0f;
  p.s16x2 = half2_of(s);
  p.s16x2b = half2_of(s_b);
  return p;
}

__device__ __forceinline__ uint4 dq_int4(unsigned w, const DqParams& p, const DqConsts<Q_INT4>& k) {
  const unsigned w8 = w >> 8;
  const unsigned u0 = (w & k.m_lo) | k.c1024;   // e0, e1: 1024 + q
  const unsigned u1 = (w & k.m_hi) | k.c64;     // e2, e3: 64 + q
  const unsigned u2 = (w8 & k.m_lo) | k.c1024;  // e4, e5
  const unsigned u3 = (w8 & k.m_hi) | k.c64;    // e6, e7
  return make_uint4(fmix2(u0, p.s, p.b1024), fmix2(u1, p.s, p.b64), fmix2(u2, p.s, p.b1024),
                    fmix2(u3, p.s, p.b64));
}

__device__ __forceinline__ uint4 dq_int8(unsigned w0, unsigned w1, const DqParams& p, const DqConsts<Q_INT8>& k) {
  // v_perm_b32: selector bytes 0..3 pick bytes of the second operand (the codes),
  // 4..7 bytes of the first (0x64): (q_e, 0x64, q_e+1, 0x64) = fp16 1024 + q
  const unsigned u0 = __builtin_amdgcn_perm(k.c64x4, w0, 0x04010400u);
  const unsigned u1 = __builtin_amdgcn_perm(k.c64x4, w0, 0x04030402u);
  const unsigned u2 = __builtin_amdgcn_perm(k.c64x4, w1, 0x04010400u);
  const unsigned u3 = __builtin_amdgcn_perm(k.c64x4, w1, 0x04030402u);
  return make_uint4(fmix2(u0, p.s, p.b1024), fmix2(u1, p.s, p.b1024), fmix2(u2, p.s, p.b1024),
                    fmix2(u3, p.s, p.b1024));
}

// Ternary chunk in layout A (LB = 0: code 2p at bit 2p, 2p+1 at 16+2p) or B
// (LB = 1: bits 8+2p, 24+2p) -> 8 fp16 weights t * fp16(s).  v_perm_b32 picks
// each value's high byte from {0xBC, 0x00, 0x3C, 0x00} (code 0 -> -1.0, 1 -> 0,
// 2 -> +1.0, 3 -> 0); selector 12 yields the zero low bytes.  SPLIT: codes 4-7
// (pairs 2, 3) take the next group's scale, s16x2b.
template <int LB, bool SPLIT = false>
__device__ __forceinline__ uint4 dq_tern(unsigned w, const DqParams& p, const DqConsts<Q_TERN>& k) {
  constexpr unsigned kTable = 0x003C00BCu;
  unsigned o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const unsigned v = LB ? (w >> (2 * q)) : (w << (8 - 2 * q));
    const unsigned sel = (v & k.t_mask) | k.t_zero;
    const unsigned t = __builtin_amdgcn_perm(0u, kTable, sel);
    half2_t th, sh;
    __builtin_memcpy(&th, &t, 4);
    __builtin_memcpy(&sh, (SPLIT && q >= 2) ? &p.s16x2b : &p.s16x2, 4);
    const half2_t r = th * sh;
    __builtin_memcpy(&o[q], &r, 4);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

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
};

}  // namespace

// ---------------------------------------------------------------------------
// The fused kernel.  QT: Q_INT4 / Q_INT8 / Q_TERN; KQ: basis functions per
// feature (1, 2, 4, 8); HB: SiLU base branch; BASIS: the A-fragment generator
// (BASIS_CHEBY_POST, BASIS_RBF_REC, BASIS_BSPLINE; see BasisGen).  Grid:
// m_tiles * n_tiles workgroups (x) by feature splits (y), 512 threads.
// ---------------------------------------------------------------------------
template <int QT, int KQ, int HB, int BASIS = BASIS_CHEBY_POST>
__global__ void __launch_bounds__(kQThreads, 1) kan_qfused_block(QPArgs A) {
  constexpr int KP = KQ + HB;
  constexpr int NV = 8;
  constexpr int SLOT = kQNB * 64;  // uint4 per slot of the N-tile
  constexpr int CB = qp_chunk_bytes(QT);
  constexpr int GS = qp_group(QT);
  constexpr int PF = qp_param_floats(QT);
  constexpr int NCB = QT == Q_TERN ? (KQ == 1 ? 1 : KQ / 2) : (KQ * CB) / 4;  // basis code dwords per block
  constexpr int NCW = QT == Q_INT8 ? 2 : 1;                                     // base code dwords
  typedef half8 frag;
  static_assert(KQ == 1 || KQ == 2 || KQ == 4 || KQ == 8, "a chunk must lie in one or two whole groups");
  // ternary at K = 8: codes 0-3 and 4-7 of a chunk in consecutive groups of 32
  constexpr bool TSPLIT = QT == Q_TERN && 8 * KQ > GS;
  constexpr int PFB = TSPLIT ? 2 : PF;  // parameter floats per basis chunk

  __shared__ uint4 stage0[KP * SLOT];
  __shared__ uint4 stage1[KP * SLOT];

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
    float pb[PFB], pw[PF];
  };
  // chunk words of segment / slot group g of feature block fbq (clamped into
  // the split: loads past it re-read the last block, in bounds).  Codes are
  // laid out [fb][ob][g][lane], one 64-lane word group per slot (ternary with
  // even K: per slot pair), so each load is one coalesced 64-lane access.
  constexpr int WB = QT == Q_TERN ? (KQ == 1 ? 2 : 4) : CB;   // bytes of one basis word group entry
  constexpr int NG = QT == Q_TERN ? (KQ == 1 ? 1 : KQ / 2) : KQ;  // basis word groups per block
  // Every address is a wave-uniform base (feature block, column block, slot
  // group) plus this lane's fixed byte offset, so the loads take the
  // scalar-base + 32-bit vector-offset form and cost no per-block VALU.
  // Group of a lane's chunk: g = (16 f + 8 hh) K / GS = 16 f K / GS + hh (8 K / GS)
  // (8 K is a multiple of GS or smaller than it, and 16 f K of 8 K): the hh
  // term is 0 for 8 K < GS, hh for 8 K = GS (INT at K = 8, ternary at K = 4)
  // and 2 hh for ternary at K = 8, whose codes 4-7 use group g + 1 (base
  // segment, K = 1: 0).
  const unsigned cb_off = (unsigned)lane * WB, cw_off = (unsigned)lane * CB;
  const unsigned pb_off = (unsigned)((((8 * KQ) / GS) * hh * M.ldp + o) * PF * 4);
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
  auto load_params = [&](int fbq, QRegs& r) __attribute__((always_inline)) {
    const int f = min(fbq, fb_end - 1);
    const char* pb = reinterpret_cast<const char*>(M.pb + (long)((16 * f * KQ) / GS) * M.ldp * PF) + pb_off;
    r.pb[0] = reinterpret_cast<const float*>(pb)[0];
    if constexpr (PF == 2) r.pb[1] = reinterpret_cast<const float*>(pb)[1];
    if constexpr (TSPLIT) r.pb[1] = reinterpret_cast<const float*>(pb + M.ldp * PF * 4)[0];  // group g + 1
    if constexpr (HB) {
      const char* pw = reinterpret_cast<const char*>(M.pw + (long)((16 * f) / GS) * M.ldp * PF) + pw_off;
      r.pw[0] = reinterpret_cast<const float*>(pw)[0];
      if constexpr (PF == 2) r.pw[1] = reinterpret_cast<const float*>(pw)[1];
    }
  };
  auto load_all = [&](int fbq, QRegs& r) {
    static_for<0, NG>([&](auto G) __attribute__((always_inline)) { load_cb(fbq, decltype(G)::value, r); });
    if constexpr (HB) load_cw(fbq, r);
    load_params(fbq, r);
  };
  // after slot SC's chunk has been decoded: refill its word (group) for block fbq
  auto reload_slot = [&](auto SCC, int fbq, QRegs& r) __attribute__((always_inline)) {
    constexpr int SC = decltype(SCC)::value;
    if constexpr (HB && SC == 0) {
      load_cw(fbq, r);
    } else {
      constexpr int k = SC - HB;
      if constexpr (QT != Q_TERN || KQ == 1) load_cb(fbq, k, r);
      else if constexpr (k & 1) load_cb(fbq, k / 2, r);  // both slots of the pair decoded
    }
  };
  // decoded chunk of slot SC (compile time) from the registers of one block
  auto dq_slot = [&](auto SCC, const QRegs& r, const DqParams& pb, const DqParams& pw)
      __attribute__((always_inline)) -> uint4 {
    constexpr int SC = decltype(SCC)::value;
    if constexpr (HB && SC == 0) {
      if constexpr (QT == Q_INT4) return dq_int4(r.cw[0], pw, dk);
      else if constexpr (QT == Q_INT8) return dq_int8(r.cw[0], r.cw[1], pw, dk);
      else return dq_tern<0>(tern_spread(r.cw[0]), pw, dk);
    } else {
      constexpr int k = SC - HB;
      if constexpr (QT == Q_INT4) return dq_int4(r.cb[k], pb, dk);
      else if constexpr (QT == Q_INT8) return dq_int8(r.cb[2 * k], r.cb[2 * k + 1], pb, dk);
      else if constexpr (KQ == 1) return dq_tern<0>(tern_spread(r.cb[0]), pb, dk);
      else return dq_tern<k & 1, TSPLIT>(r.cb[k / 2], pb, dk);
    }
  };
  auto params_of = [&](const QRegs& r, DqParams& pb, DqParams& pw) {
    if constexpr (QT == Q_TERN) {
      pb = dq_params_tern(r.pb[0], r.pb[PFB - 1]);
      if constexpr (HB) pw = dq_params_tern(r.pw[0], r.pw[0]);
    } else {
      pb = dq_params_affine(r.pb[0], r.pb[1]);
      if constexpr (HB) pw = dq_params_affine(r.pw[0], r.pw[1]);
    }
  };
  // Features 16 fbq + 8 (lane / 32) + e at or past D_in must contribute zero
  // weights (their affine group parameters belong to real features too): in
  // the last feature block of a ragged D_in (a wave-uniform condition) the
  // decoded halves of those features are cleared.
  auto is_tail = [&](int fbq) -> bool { return 16 * (min(fbq, fb_end - 1) + 1) > D_in; };
  auto mask_tail = [&](int fbq, uint4& v) {
    const int nv = max(0, min(8, D_in - (16 * min(fbq, fb_end - 1) + 8 * hh)));
    v.x &= (0 < nv ? 0x0000FFFFu : 0u) | (1 < nv ? 0xFFFF0000u : 0u);
    v.y &= (2 < nv ? 0x0000FFFFu : 0u) | (3 < nv ? 0xFFFF0000u : 0u);
    v.z &= (4 < nv ? 0x0000FFFFu : 0u) | (5 < nv ? 0xFFFF0000u : 0u);
    v.w &= (6 < nv ? 0x0000FFFFu : 0u) | (7 < nv ? 0xFFFF0000u : 0u);
  };

  // ---- inputs (as kan_fused_block): lane holds x[row0 + lane%32][16 fb + 8 (lane/32) + j]
  uint4 xr[2];
  auto xload = [&](int fbx) {
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
  auto xunpack = [&](int fbx, float* xf) {
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
  auto pack = [&](frag& a, const float* v) {
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = (_Float16)v[j];
  };
  auto bread = [&](frag (&b)[kQNB], const uint4* stage, int s) {
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
  load_all(fb_begin, R);
  xload(fb_begin);
  {
    DqParams pb, pw;
    params_of(R, pb, pw);
    const bool tail = is_tail(fb_begin);
    uint4 v[KP];
    static_for<0, KP>([&](auto SCC) __attribute__((always_inline)) {
      constexpr int SC = decltype(SCC)::value;
      v[SC] = dq_slot(SCC, R, pb, pw);
      if (tail) mask_tail(fb_begin, v[SC]);
    });
    load_all(fb_begin + 1, R);
#pragma unroll
    for (int sc = 0; sc < KP; ++sc) stage0[(sc * kQNB + wave) * 64 + lane] = v[sc];
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

  // One feature block: MFMAs of block fb from `cur`, decode of block fb + 1 (in
  // R) into `nxt`, R refilled with block fb + 2.
  auto block = [&](int fb, const uint4* cur, uint4* nxt) __attribute__((always_inline)) {
    float xf[NV];
    xunpack(fb, xf);
    if (fb + 1 < fb_end) xload(fb + 1);
    DqParams pb, pw;
    params_of(R, pb, pw);
    const bool tail = is_tail(fb + 1);
    load_params(fb + 2, R);
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
      // decode slot SC of block fb + 1, then refill its code word with block fb + 2
      const uint4 d = dq_slot(SCC, R, pb, pw);
      reload_slot(SCC, fb + 2, R);
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
        mask_tail(fb + 1, v);
        nxt[(sc * kQNB + wave) * 64 + lane] = v;
      }
    }
    // the decoded block is in LDS (lgkmcnt(0)) and every wave is done with `cur`;
    // the register loads stay in flight across the barrier
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  for (int fb = fb_begin; fb < fb_end; fb += 2) {
    block(fb, stage0, stage1);
    if (fb + 1 < fb_end) block(fb + 1, stage1, stage0);
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
  // one thread per (fb, ob, slot pair, lane) for even Kseg, per (fb, ob, lane) for Kseg = 1
  const int per = Kseg == 1 ? 1 : Kseg / 2;
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
      if (o >= D_out || i >= D_in) return 1u;  // zero weight
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
  const long n = (long)nfb * nob_pad * 64 * (Kseg == 1 ? 1 : Kseg / 2);
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

template <int QT, int KQ, int HB, int BASIS>
static void qp_go(const QPArgs& A, dim3 grid, hipStream_t st) {
  hipLaunchKernelGGL((kan_qfused_block<QT, KQ, HB, BASIS>), grid, dim3(kQThreads), 0, st, A);
}

// Instantiated (QT, K, basis) combinations: qp_supported.
template <int QT, int BASIS>
static hipError_t qp_dispatch_k(const QPLaunch& L, const QPArgs& A, dim3 grid, hipStream_t st) {
#define QP_K(KV)                                                   \
  if (L.K == KV) {                                                 \
    if (L.has_base) qp_go<QT, KV, 1, BASIS>(A, grid, st);          \
    else qp_go<QT, KV, 0, BASIS>(A, grid, st);                     \
    return hipGetLastError();                                      \
  }
  if constexpr (BASIS == BASIS_CHEBY_POST) {
    QP_K(1)
    QP_K(2)
  }
  if constexpr (BASIS != BASIS_BSPLINE_TAB) QP_K(4)
  if constexpr (BASIS != BASIS_BSPLINE && !(QT == Q_INT8 && BASIS == BASIS_BSPLINE_TAB)) QP_K(8)
#undef QP_K
  return hipErrorInvalidValue;
}

template <int QT>
static hipError_t qp_dispatch_basis(const QPLaunch& L, const QPArgs& A, dim3 grid, hipStream_t st) {
  switch (L.basis) {
    case BASIS_CHEBY: return qp_dispatch_k<QT, BASIS_CHEBY_POST>(L, A, grid, st);
    case BASIS_RBF: return qp_dispatch_k<QT, BASIS_RBF_REC>(L, A, grid, st);
    default:  // G = 5 (K = 8): the basis table; K = 4 (G = 1): per-value selection
      if (L.K == kBsplineTabG + 3) return qp_dispatch_k<QT, BASIS_BSPLINE_TAB>(L, A, grid, st);
      return qp_dispatch_k<QT, BASIS_BSPLINE>(L, A, grid, st);
  }
}

hipError_t qp_launch(const QPLaunch& L, hipStream_t st) {
  if (!qp_supported(L.qt, L.K, L.basis, L.bp.rbf_rec) || (L.grp != 4 && L.grp != 8) || L.B <= 0 ||
      (L.basis != BASIS_CHEBY && (L.grp != 8 || L.bp.K != L.K)))
    return hipErrorInvalidValue;
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
  A.m_tiles = (L.B + 255) / 256;
  A.n_tiles = (L.m[0].D_out + 32 * L.grp - 1) / (32 * L.grp);
  A.nfb = (L.D_in + 15) / 16;
  const int splits = std::max(1, std::min(L.splits, A.nfb));
  A.fb_per_split = (A.nfb + splits - 1) / splits;
  const int nsp = (A.nfb + A.fb_per_split - 1) / A.fb_per_split;
  A.part = nsp > 1 ? L.part : nullptr;
  A.epi = L.epi;
  A.round16 = L.round16;
  A.bp = L.bp;
  const dim3 grid((unsigned)(A.m_tiles * A.n_tiles), (unsigned)nsp);
  hipError_t e;
  switch (L.qt) {
    case Q_INT4: e = qp_dispatch_basis<Q_INT4>(L, A, grid, st); break;
    case Q_INT8: e = qp_dispatch_basis<Q_INT8>(L, A, grid, st); break;
    default: e = qp_dispatch_basis<Q_TERN>(L, A, grid, st); break;
  }
  if (e != hipSuccess || nsp <= 1) return e;
  const long n = (long)L.B * L.m[0].D_out;
  hipLaunchKernelGGL(k_qp_finalize, dim3(grid_of(n)), dim3(256), 0, st, (const float*)L.part, nsp, L.B, A.n_tiles,
                     L.epi, L.grp, L.m[0].bias, L.grp == 4 ? L.m[1].bias : nullptr, L.bias_dtype, L.m[0].D_out, L.Y,
                     L.ldy, L.y_dtype, L.round16);
  return hipGetLastError();
}

}  // namespace kans
