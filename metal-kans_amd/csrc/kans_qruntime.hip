// Runtime objects of the quantized paths: a KAN layer (Chebyshev, RBF or
// B-spline basis) held in the reference's packed INT8 / INT4 / ternary formats
// (kans_qlayer) and the GatedKAN block of three such layers (kans_gated), plus
// the reference-named fused ternary entry point.  Batches of at most 32 rows
// take the decode GEMVs (kans_qgemv.hip, every format); larger batches the
// fused prefill kernel (kans_qprefill_kernel.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <map>
#include <cstring>
#include <vector>

#include "kans_api_internal.h"
#include "kans_qgemv.h"
#include "kans_qprefill.h"

using namespace kans;

namespace kans {
int dequant_ternary_device(const uint32_t* p, const float* s, float* out, int D_out, int K_dim, int gs,
                           hipStream_t st);
}

struct kans_qlayer {
  int quant;                 // Q_INT4 / Q_TERN / Q_INT8
  int D_in, D_out, K, has_base, has_bias, group;
  int basis = BASIS_CHEBY;   // basis expansion (kans_qlayer_set_rbf / _bspline; Chebyshev by default)
  BasisParams bp{};          // its parameters (bp.K = K)
  int Cb, Cw, C_tot;         // superchunks: basis, base, total
  int nw;                    // 16-row blocks per decode row group (qrow_blocks)
  int nrb_pad;               // 16-row blocks, padded to a multiple of nw
  bool decode = false;       // decode records built (INT4 / ternary)
  DevBuf R, bias;            // re-tiled records (codes + group parameters), bias (bias_dtype)
  int bias_dtype = DT_F32;
  // decode workspace: activation basis, its group sums, split-K partials
  DevBuf Phi, S, part;
  DevBuf cnt;                // arrival counters of the fused epilogue, one per row group, kCntStride ints
                             // apart (0 between launches)
  // prefill tiles (kans_qprefill.h): codes and group parameters of the basis and base segments
  bool prefill = false;
  int p_nfb = 0, p_nob_pad = 0;
  DevBuf PCb, PCw, PPb, PPw;
  DevBuf p_part;             // prefill split workspace
  DevBuf hx, hy;             // staging of the host-pointer forward (grow-only)
};

struct kans_gated {
  kans_qlayer *gate, *up, *down;
  DevBuf hidden;  // SwiGLU(gate, up): [B][h] fp32 (decode, separate kernels) or [B][ld_h] (prefill)
  DevBuf p_part;  // prefill split workspace
  DevBuf hx, hy;  // staging of the host-pointer forward (grow-only)
};

namespace {

constexpr int kMaxDecodeB = 32;

// GatedKAN: SwiGLU and the down layer's basis in one step -- the gate|up
// GEMV's epilogue (QEPI_SWIGLU) at B <= 2, k_swiglu_basis above -- instead of
// k_qswiglu + k_prep.
bool g_fused_swiglu = true;
// In-kernel basis of x in the gate|up GEMV (kans_decode_set_pre_basis): 0 never,
// 1 at B = 1, 2 at B <= 2.  At B = 2 the waves' longer basis phase (two rows)
// outweighs the launch it saves: cfg5 block at B = 2, INT4 93.5 against
// 87.2 us with k_prep, ternary 68.4 / 64.5, INT8 150.9 / 149.0; at B = 1 it
// gains (INT4 82.1 / 82.8, ternary 60.1 / 61.6, INT8 141.8 / 144.8; one box,
// three runs each).
int g_pre_basis = 1;

int mp_of(int B) { return B <= 16 ? 16 : 32; }

size_t dt_bytes(int dt) { return dt == DT_F32 ? 4 : 2; }

// Weight-record loads of the decode GEMVs: 0 automatic (use_nt), 1 plain,
// 2 non-temporal.
int g_weight_loads = 0;

// Packed bytes of a layer's re-tiled records (codes + group parameters).
size_t rec_bytes(const kans_qlayer* L) {
  return (size_t)(L->nrb_pad / L->nw) * L->C_tot * qrec_bytes(L->quant);
}

// Cache policy of the weight-record loads.  A decode step of a model streams
// every layer's weights once, and a model whose quantized layers together
// exceed the 256 MB MALL finds none of them cached on its next step, so the
// choice is made for weights read from HBM: measured on the config-5 blocks,
// three weight copies chained in one decode-step graph (one box, same run,
// us per block, non-temporal / plain):
//   INT4    B = 1: 75.2 / 83.9;  B = 32: 122.3 / 127.9
//   ternary B = 1: 52.6 / 57.2;  B = 32: 94.3 / 98.7
//   INT8    B = 1: 122.1 / 136.4; B = 32: 167.7 / 180.1
// so every format loads non-temporally.  (With each lane's 32 INT8 bytes
// contiguous, so that each 16-byte load covered half of every cache line of
// the tile, non-temporal loads were the slower form for INT8: 145.2 / 136.5
// at B = 1.  A ternary block replayed alone stays in the MALL and is faster
// with plain loads, but that is not how a model's layers are read.)
int use_nt(int /*quant*/) {
  if (g_weight_loads != 0) return g_weight_loads == 2 ? 1 : 0;
  return 1;
}

// Superchunk ranges per row group: about items_per_cu work items (waves) per
// CU, at least 4 superchunks per item.
int choose_ksplit(int n_rg, int C_tot, int B, int quant) {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
      cus = prop.multiProcessorCount;
    if (cus <= 0) cus = 256;
  }
  const int per_cu = items_per_cu(quant, B);
  int ks = B <= kSmallB ? per_cu * cus / n_rg : (per_cu * cus + n_rg - 1) / n_rg;
  ks = std::min(ks, std::max(1, C_tot / 4));
  return std::max(ks, 1);
}

int layer_geometry(kans_qlayer* L) {
  const long Jb = (long)L->D_in * L->K;
  if (q_affine(L->quant)) {
    const long pb = (Jb + L->group - 1) / L->group * L->group;
    const long pw = ((long)L->D_in + L->group - 1) / L->group * L->group;
    L->Cb = (int)((pb + kQSuper - 1) / kQSuper);
    L->Cw = L->has_base ? (int)((pw + kQSuper - 1) / kQSuper) : 0;
  } else {
    L->Cb = (int)((Jb + kQSuper - 1) / kQSuper);
    L->Cw = L->has_base ? (int)(((long)L->D_in + kQSuper - 1) / kQSuper) : 0;
  }
  L->C_tot = L->Cb + L->Cw;
  L->nw = qrow_blocks(L->D_out);
  L->nrb_pad = round_up((L->D_out + 15) / 16, L->nw);
  return 0;
}

int validate_q(int D_in, int D_out, int K, int has_base, int has_bias, int group, int quant) {
  if (D_in <= 0 || D_out <= 0 || K <= 0 || K > kMaxK)
    return kans_fail(KANS_ERR_ARG, "bad dims D_in=%d D_out=%d K=%d", D_in, D_out, K);
  if ((has_base != 0 && has_base != 1) || (has_bias != 0 && has_bias != 1))
    return kans_fail(KANS_ERR_ARG, "has_base/has_bias must be 0 or 1");
  if ((quant == Q_INT4 || quant == Q_INT8) && group != 64)
    return kans_fail(KANS_ERR_UNSUPPORTED, "fused INT%d path needs group_size 64 (got %d)", quant == Q_INT8 ? 8 : 4,
                     group);
  if (quant == Q_TERN && group != 32)
    return kans_fail(KANS_ERR_UNSUPPORTED, "fused ternary path needs group_size 32 (got %d)", group);
  return 0;
}

// Upload host bytes to a temporary device buffer.
int upload_tmp(DevBuf& d, const void* src, size_t bytes, hipStream_t st) {
  int rc = d.reserve(bytes ? bytes : 16);
  if (rc) return rc;
  if (bytes) HIP_TRY(hipMemcpyAsync(d.p, src, bytes, hipMemcpyHostToDevice, st));
  return 0;
}

// Prefill tiles of one segment (seg 0: basis, K per feature; seg 1: base, one per feature) from
// the reference arrays already on the device.
int build_ptiles(kans_qlayer* L, int seg, const void* codes, long rowbytes, const float* scales,
                 const float* biases, int gpr, hipStream_t st) {
  const int Kseg = seg ? 1 : L->K;
  const int CB = qp_chunk_bytes(L->quant), GS = qp_group(L->quant), PF = qp_param_floats(L->quant);
  // ternary pads an odd Kseg > 1 to whole slot pairs
  const int Kpad = L->quant == Q_TERN && Kseg > 1 ? (Kseg + 1) / 2 * 2 : Kseg;
  const size_t cbytes = (size_t)L->p_nfb * L->p_nob_pad * 64 * Kpad * CB;
  // groups of every index, plus zero rows for the kernel's loads of a
  // half-block's later groups (up to 3 past the first) and of its first group
  // (qp_gl, up to 2 past the block's)
  const int G_alloc = (16 * L->p_nfb * Kseg + GS - 1) / GS + 6;
  const long ldp = (long)L->p_nob_pad * 32;
  DevBuf& C = seg ? L->PCw : L->PCb;
  DevBuf& P = seg ? L->PPw : L->PPb;
  int rc = C.reserve(cbytes);
  if (rc) return rc;
  if ((rc = P.reserve((size_t)G_alloc * ldp * PF * sizeof(float)))) return rc;
  hipError_t e;
  if (L->quant == Q_TERN)
    e = qp_tile_tern((const unsigned*)codes, (int)rowbytes, scales, gpr, L->D_out, L->D_in, Kseg, L->p_nfb,
                     L->p_nob_pad, G_alloc, C.p, (float*)P.p, st);
  else
    e = qp_tile_affine(L->quant == Q_INT8 ? 8 : 4, (const unsigned char*)codes, rowbytes, scales, biases, gpr,
                       L->D_out, L->D_in, Kseg, L->p_nfb, L->p_nob_pad, G_alloc, C.p, (float*)P.p, st);
  if (e != hipSuccess) return kans_fail(KANS_ERR_HIP, "prefill re-tiling failed: %s", hipGetErrorString(e));
  return 0;
}

void prefill_geometry(kans_qlayer* L) {
  L->prefill = qp_supported(L->quant, L->K, L->has_base);
  L->p_nfb = (L->D_in + 15) / 16;
  L->p_nob_pad = round_up((L->D_out + 31) / 32, 8);
}

QPMat qp_mat(const kans_qlayer* L) {
  QPMat m;
  m.cb = (const unsigned char*)L->PCb.p;
  m.cw = (const unsigned char*)L->PCw.p;
  m.pb = (const float*)L->PPb.p;
  m.pw = (const float*)L->PPw.p;
  m.ldp = (long)L->p_nob_pad * 32;
  m.nob_pad = L->p_nob_pad;
  m.D_out = L->D_out;
  m.bias = L->has_bias ? L->bias.p : nullptr;
  return m;
}

int alloc_tiles(kans_qlayer* L) {
  const size_t bytes = (size_t)(L->nrb_pad / L->nw) * L->C_tot * qrec_bytes(L->quant);
  int rc = L->R.reserve(bytes);
  if (rc) return rc;
  HIP_TRY(hipMemsetAsync(L->R.p, 0, bytes, kans_default_stream()));
  const size_t cbytes = (size_t)(L->nrb_pad / L->nw) * kCntStride * sizeof(int);
  if ((rc = L->cnt.reserve(cbytes))) return rc;
  HIP_TRY(hipMemsetAsync(L->cnt.p, 0, cbytes, kans_default_stream()));
  return 0;
}

int upload_bias(kans_qlayer* L, const void* bias, int bias_dtype) {
  if (!L->has_bias) return 0;
  if (!bias) return kans_fail(KANS_ERR_ARG, "has_bias set but bias is null");
  if (bias_dtype < DT_F32 || bias_dtype > DT_BF16) return kans_fail(KANS_ERR_ARG, "bad bias dtype %d", bias_dtype);
  const size_t bytes = (size_t)L->D_out * (bias_dtype == DT_F32 ? 4 : 2);
  int rc = L->bias.reserve(bytes);
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(L->bias.p, bias, bytes, hipMemcpyHostToDevice, kans_default_stream()));
  L->bias_dtype = bias_dtype;
  return 0;
}

// Device workspace of one decode forward: the activation basis (Phi, S) and the
// split-K partial sums of each GEMV (the layer's, or gate|up then down), the
// fused epilogue's arrival counters (0 between launches) and, with the
// separate-kernel SwiGLU, the hidden state.
struct DecodeWS {
  _Float16* phi = nullptr;
  float2* s = nullptr;
  float* part = nullptr;
  _Float16* phi2 = nullptr;
  float2* s2 = nullptr;
  float* part2 = nullptr;
  int* cnt = nullptr;
  float* hidden = nullptr;
};

size_t phi_bytes(const kans_qlayer* L, int B) { return (size_t)mp_of(B) * L->C_tot * kQSuper * sizeof(_Float16); }
size_t s_bytes(const kans_qlayer* L, int B) { return (size_t)L->C_tot * mp_of(B) * sizeof(float2); }
size_t part_bytes(int B, int ksplit, int N_total) { return (size_t)ksplit * B * N_total * sizeof(float); }

int reserve_decode(kans_qlayer* L, int B, int ksplit, int N_total) {
  int rc = L->Phi.reserve(phi_bytes(L, B));
  if (rc) return rc;
  if ((rc = L->S.reserve(s_bytes(L, B)))) return rc;
  return L->part.reserve(part_bytes(B, ksplit, N_total));
}

int prep_locked(kans_qlayer* L, const void* X, int x_dtype, long ldx, int B, _Float16* phi, float2* S,
                hipStream_t st) {
  QPrep P;
  P.X = X;
  P.x_dtype = x_dtype;
  P.ldx = ldx;
  P.B = B;
  P.MP = mp_of(B);
  P.D_in = L->D_in;
  P.K = L->K;
  P.has_base = L->has_base;
  P.Cb = L->Cb;
  P.C_tot = L->C_tot;
  P.Phi = phi;
  P.S = S;
  P.basis = L->basis;
  P.bp = L->bp;
  HIP_TRY(qprep(L->quant, P, st));
  return 0;
}

// Whether the fused prefill kernel covers this layer (tiles built, K and basis instantiated).
bool prefill_ok(const kans_qlayer* L) {
  return L->prefill && qp_supported(L->quant, L->K, L->has_base, L->basis, L->bp.rbf_rec);
}

// GEMV of layer a (and b, sharing a's activations phi / S): split-K partial sums
// in part ([ksplit][B][a.D_out + b.D_out]), then the epilogue `epi`.
int gemv_locked(kans_qlayer* a, kans_qlayer* b, int B, int ksplit, const QEpi& epi, int nt, const _Float16* phi,
                const float2* S, float* part, hipStream_t st, const void* X = nullptr, int x_dtype = 0,
                long ldx = 0) {
  QGemv G;
  if (X) {  // in-kernel basis of a's input (qgemv_pre_fits checked by the caller)
    G.X = X;
    G.x_dtype = x_dtype;
    G.ldx = ldx;
    G.D_in = a->D_in;
    G.K = a->K;
    G.has_base = a->has_base;
    G.Cb = a->Cb;
  }
  G.rec0 = a->R.p;
  G.D_out0 = a->D_out;
  G.rec1 = b ? b->R.p : nullptr;
  G.D_out1 = b ? b->D_out : 0;
  G.nw = a->nw;
  G.rg_split = a->nrb_pad / a->nw;
  G.n_rg = G.rg_split + (b ? b->nrb_pad / b->nw : 0);
  G.ksplit = ksplit;
  G.C_tot = a->C_tot;
  G.Phi = phi;
  G.S = S;
  G.B = B;
  G.MP = mp_of(B);
  G.part = part;
  G.N_total = a->D_out + (b ? b->D_out : 0);
  G.epi = epi;
  G.nt = nt;
  HIP_TRY(qgemv(a->quant, G, st));
  return 0;
}

// GEMV of layer L on its prepared phi / S, then the split-K reduce + bias into Y.
int gemv_reduce_locked(kans_qlayer* L, int B, int ks, void* Y, int y_dtype, long ldy, int nt, const _Float16* phi,
                       const float2* S, float* part, hipStream_t st) {
  int rc = gemv_locked(L, nullptr, B, ks, QEpi{}, nt, phi, S, part, st);
  if (rc) return rc;
  HIP_TRY(qreduce(part, ks, B, L->D_out, L->has_bias ? L->bias.p : nullptr, L->bias_dtype, Y, y_dtype, ldy, st));
  return 0;
}

int check_x(const void* X, int x_dtype, long ldx, int D_in, int B) {
  if (!X) return kans_fail(KANS_ERR_ARG, "null X");
  if (x_dtype < DT_F32 || x_dtype > DT_BF16) return kans_fail(KANS_ERR_ARG, "bad x dtype %d", x_dtype);
  if (ldx < D_in) return kans_fail(KANS_ERR_ARG, "ldx=%ld < D_in=%d", ldx, D_in);
  if (B <= 0 || B > kMaxDecodeB) return kans_fail(KANS_ERR_ARG, "decode path takes 1 <= B <= %d (got %d)", kMaxDecodeB, B);
  return 0;
}

// Input of the fused prefill kernel: fp16 or fp32 rows, 16-byte aligned, ldx a
// multiple of 8 and >= round_up(D_in, 8) (the kernel reads whole 8-feature
// chunks and ignores the columns past D_in).
int check_prefill_x(const void* X, int x_dtype, long ldx, int D_in) {
  if (!X) return kans_fail(KANS_ERR_ARG, "null X");
  if (x_dtype != DT_F16 && x_dtype != DT_F32)
    return kans_fail(KANS_ERR_UNSUPPORTED, "prefill path reads fp16 or fp32 inputs (x dtype %d)", x_dtype);
  if (ldx < round_up(D_in, 8) || ldx % 8 != 0)
    return kans_fail(KANS_ERR_ARG, "prefill path needs ldx %% 8 == 0 and ldx >= %d (got %ld)", round_up(D_in, 8), ldx);
  if (((uintptr_t)X & 15) != 0) return kans_fail(KANS_ERR_ARG, "prefill path needs a 16-byte aligned X");
  return 0;
}

int check_y(const void* Y, int y_dtype, long ldy, int D_out) {
  if (!Y || ldy < D_out) return kans_fail(KANS_ERR_ARG, "bad Y / ldy");
  if (y_dtype < DT_F32 || y_dtype > DT_BF16) return kans_fail(KANS_ERR_ARG, "bad y dtype %d", y_dtype);
  return 0;
}

// Fused prefill forward of one layer (kans_qprefill_kernel.h), any batch.
int prefill_layer_locked(kans_qlayer* L, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy, int B,
                         hipStream_t st) {
  if (!prefill_ok(L))
    return kans_fail(KANS_ERR_UNSUPPORTED,
                     "the fused quantized prefill path takes Chebyshev K <= 9, RBF on uniform centres 2 <= K <= 9 and "
                     "B-spline K in {4, 8} (not INT8 with the base branch at K = 7, nor INT8 B-spline at K = 8); this "
                     "layer has K = %d, basis %d", L->K, L->basis);
  int rc = check_prefill_x(X, x_dtype, ldx, L->D_in);
  if (rc) return rc;
  QPLaunch P{};
  P.qt = L->quant;
  P.K = L->K;
  P.has_base = L->has_base;
  P.basis = L->basis;
  P.bp = L->bp;
  P.X = X;
  P.ldx = ldx;
  P.x_dtype = x_dtype;
  P.m[0] = qp_mat(L);
  P.m[1] = P.m[0];
  P.grp = 8;
  P.bias_dtype = L->bias_dtype;
  P.Y = Y;
  P.ldy = ldy;
  P.y_dtype = y_dtype;
  P.B = B;
  P.D_in = L->D_in;
  P.splits = qp_choose_splits(B, L->D_in, L->D_out, 8);
  P.epi = QP_EPI_PLAIN;
  const long pf = qp_part_floats(P);
  if (pf > 0) {
    if ((rc = L->p_part.reserve((size_t)pf * sizeof(float)))) return rc;
    P.part = (float*)L->p_part.p;
  }
  HIP_TRY(qp_launch(P, st));
  return 0;
}

int qlayer_forward_locked(kans_qlayer* L, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy, int B,
                          hipStream_t st) {
  int rc = check_y(Y, y_dtype, ldy, L->D_out);
  if (rc) return rc;
  if (B < 0) return kans_fail(KANS_ERR_ARG, "B=%d < 0", B);
  if (B == 0) return 0;
  if (B > kMaxDecodeB || !L->decode) return prefill_layer_locked(L, X, x_dtype, ldx, Y, y_dtype, ldy, B, st);
  if ((rc = check_x(X, x_dtype, ldx, L->D_in, B))) return rc;
  const int ks = choose_ksplit(L->nrb_pad / L->nw, L->C_tot, B, L->quant);
  if ((rc = reserve_decode(L, B, ks, L->D_out))) return rc;
  _Float16* phi = (_Float16*)L->Phi.p;
  float2* S = (float2*)L->S.p;
  if ((rc = prep_locked(L, X, x_dtype, ldx, B, phi, S, st))) return rc;
  return gemv_reduce_locked(L, B, ks, Y, y_dtype, ldy, use_nt(L->quant), phi, S, (float*)L->part.p, st);
}

// GatedKAN prefill: one launch for gate | up with the SwiGLU epilogue into the
// hidden buffer (fp16 when round16 = 1, fp32 otherwise), one for down.
// The two launches of a GatedKAN prefill forward, and the workspace they need.
struct GatedPrefill {
  QPLaunch P1, P2;
  size_t hidden_bytes = 0, part_bytes = 0;
};

int plan_gated_prefill(kans_gated* G, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy, int B,
                       int round16, GatedPrefill& GP) {
  kans_qlayer *g = G->gate, *u = G->up, *d = G->down;
  if (!prefill_ok(g) || !prefill_ok(u) || !prefill_ok(d))
    return kans_fail(KANS_ERR_UNSUPPORTED,
                     "the fused quantized prefill path takes K <= 9 (not INT8 with the base branch at K = 7): K = %d, %d",
                     g->K, d->K);
  if (g->has_bias && u->has_bias && g->bias_dtype != u->bias_dtype)
    return kans_fail(KANS_ERR_UNSUPPORTED, "gate and up biases of different dtypes");
  int rc = check_prefill_x(X, x_dtype, ldx, g->D_in);
  if (rc) return rc;
  const int h = g->D_out;
  const long ldh = round_up(h, 8);
  const int hdt = round16 == 1 ? DT_F16 : DT_F32;
  QPLaunch& P1 = GP.P1;
  QPLaunch& P2 = GP.P2;
  P1 = QPLaunch{};
  P1.qt = g->quant;
  P1.K = g->K;
  P1.has_base = g->has_base;
  P1.X = X;
  P1.ldx = ldx;
  P1.x_dtype = x_dtype;
  P1.m[0] = qp_mat(g);
  P1.m[1] = qp_mat(u);
  P1.grp = 4;
  P1.bias_dtype = g->has_bias ? g->bias_dtype : u->bias_dtype;
  P1.ldy = ldh;
  P1.y_dtype = hdt;
  P1.B = B;
  P1.D_in = g->D_in;
  P1.splits = qp_choose_splits(B, g->D_in, h, 4);
  P1.epi = QP_EPI_SWIGLU;
  P1.round16 = round16;
  P2 = QPLaunch{};
  P2.qt = d->quant;
  P2.K = d->K;
  P2.has_base = d->has_base;
  P2.ldx = ldh;
  P2.x_dtype = hdt;
  P2.m[0] = qp_mat(d);
  P2.m[1] = P2.m[0];
  P2.grp = 8;
  P2.bias_dtype = d->bias_dtype;
  P2.Y = Y;
  P2.ldy = ldy;
  P2.y_dtype = y_dtype;
  P2.B = B;
  P2.D_in = h;
  P2.splits = qp_choose_splits(B, h, d->D_out, 8);
  P2.epi = QP_EPI_PLAIN;
  GP.hidden_bytes = (size_t)B * ldh * dt_bytes(hdt);
  GP.part_bytes = (size_t)std::max(qp_part_floats(P1), qp_part_floats(P2)) * sizeof(float);
  return 0;
}

// Enqueue a planned prefill forward with its workspace (part may be null when unsplit).
int run_gated_prefill(GatedPrefill& GP, void* hidden, float* part, hipStream_t st) {
  GP.P1.Y = hidden;
  GP.P2.X = hidden;
  GP.P1.part = GP.P2.part = part;
  HIP_TRY(qp_launch(GP.P1, st));
  HIP_TRY(qp_launch(GP.P2, st));
  return 0;
}

int prefill_gated_locked(kans_gated* G, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy, int B,
                         int round16, hipStream_t st) {
  GatedPrefill GP;
  int rc = plan_gated_prefill(G, X, x_dtype, ldx, Y, y_dtype, ldy, B, round16, GP);
  if (rc) return rc;
  if ((rc = G->hidden.reserve(GP.hidden_bytes))) return rc;
  if (GP.part_bytes && (rc = G->p_part.reserve(GP.part_bytes))) return rc;
  return run_gated_prefill(GP, G->hidden.p, GP.part_bytes ? (float*)G->p_part.p : nullptr, st);
}

// Decode GEMV split-K of the gated block's two GEMVs for batch B.
void gated_ksplits(const kans_gated* G, int B, int* ks1, int* ks2) {
  const kans_qlayer *g = G->gate, *u = G->up, *d = G->down;
  *ks1 = choose_ksplit((g->nrb_pad + u->nrb_pad) / g->nw, g->C_tot, B, g->quant);
  *ks2 = choose_ksplit(d->nrb_pad / d->nw, d->C_tot, B, d->quant);
}

// The decode forward of a gated block (1 <= B <= 32) on the workspace ws (sized for B, ks1, ks2).
int gated_decode(kans_gated* G, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy, int B,
                 int round16, int ks1, int ks2, const DecodeWS& ws, hipStream_t st) {
  kans_qlayer *g = G->gate, *u = G->up, *d = G->down;
  const int h = g->D_out;
  int rc;
  const int nt = use_nt(g->quant);
  // B = 1 (g_pre_basis) with the fused epilogue: the gate|up GEMV computes the
  // basis of x itself (no k_prep launch) when its LDS slices fit
  if (g_fused_swiglu && B <= (g_pre_basis == 2 ? kSmallB : g_pre_basis == 1 ? 1 : 0) && ks1 <= kMaxEpiSplit &&
      qgemv_pre_fits(g->quant, B, g->C_tot, ks1, QEPI_SWIGLU)) {
    QEpi e1;
    e1.kind = QEPI_SWIGLU;
    e1.counters = ws.cnt;
    e1.bias = g->has_bias ? g->bias.p : nullptr;
    e1.bias_dtype = g->bias_dtype;
    e1.bias_u = u->has_bias ? u->bias.p : nullptr;
    e1.bias_u_dtype = u->bias_dtype;
    e1.round16 = round16;
    e1.K2 = d->K;
    e1.has_base2 = d->has_base;
    e1.Cb2 = d->Cb;
    e1.C_tot2 = d->C_tot;
    e1.Phi2 = ws.phi2;
    e1.S2 = ws.s2;
    if ((rc = gemv_locked(g, u, B, ks1, e1, nt, nullptr, nullptr, ws.part, st, X, x_dtype, ldx))) return rc;
    return gemv_reduce_locked(d, B, ks2, Y, y_dtype, ldy, nt, ws.phi2, ws.s2, ws.part2, st);
  }
  if ((rc = prep_locked(g, X, x_dtype, ldx, B, ws.phi, ws.s, st))) return rc;
  if (g_fused_swiglu) {
    // SwiGLU(gate, up) straight into the down layer's basis: in the gate|up
    // GEMV's epilogue at B <= 2, by k_swiglu_basis after it otherwise
    QEpi e1;
    e1.kind = QEPI_SWIGLU;
    e1.counters = ws.cnt;
    e1.bias = g->has_bias ? g->bias.p : nullptr;
    e1.bias_dtype = g->bias_dtype;
    e1.bias_u = u->has_bias ? u->bias.p : nullptr;
    e1.bias_u_dtype = u->bias_dtype;
    e1.round16 = round16;
    e1.K2 = d->K;
    e1.has_base2 = d->has_base;
    e1.Cb2 = d->Cb;
    e1.C_tot2 = d->C_tot;
    e1.Phi2 = ws.phi2;
    e1.S2 = ws.s2;
    if (B <= kSmallB && ks1 <= kMaxEpiSplit) {
      if ((rc = gemv_locked(g, u, B, ks1, e1, nt, ws.phi, ws.s, ws.part, st))) return rc;
    } else {
      if ((rc = gemv_locked(g, u, B, ks1, QEpi{}, nt, ws.phi, ws.s, ws.part, st))) return rc;
      HIP_TRY(qswiglu_basis(g->quant, e1, ws.part, ks1, B, mp_of(B), h, st));
    }
    return gemv_reduce_locked(d, B, ks2, Y, y_dtype, ldy, nt, ws.phi2, ws.s2, ws.part2, st);
  }
  if ((rc = gemv_locked(g, u, B, ks1, QEpi{}, nt, ws.phi, ws.s, ws.part, st))) return rc;
  HIP_TRY(qswiglu(ws.part, ks1, B, h, g->has_bias ? g->bias.p : nullptr, g->bias_dtype,
                  u->has_bias ? u->bias.p : nullptr, u->bias_dtype, round16, ws.hidden, st));
  if ((rc = prep_locked(d, ws.hidden, DT_F32, h, B, ws.phi2, ws.s2, st))) return rc;
  return gemv_reduce_locked(d, B, ks2, Y, y_dtype, ldy, nt, ws.phi2, ws.s2, ws.part2, st);
}

int gated_forward_locked(kans_gated* G, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy, int B,
                         int round16, hipStream_t st) {
  kans_qlayer *g = G->gate, *u = G->up, *d = G->down;
  int rc = check_y(Y, y_dtype, ldy, d->D_out);
  if (rc) return rc;
  if (B < 0) return kans_fail(KANS_ERR_ARG, "B=%d < 0", B);
  if (B == 0) return 0;
  if (B > kMaxDecodeB || !g->decode)
    return prefill_gated_locked(G, X, x_dtype, ldx, Y, y_dtype, ldy, B, round16, st);
  if ((rc = check_x(X, x_dtype, ldx, g->D_in, B))) return rc;
  int ks1, ks2;
  gated_ksplits(G, B, &ks1, &ks2);
  if ((rc = reserve_decode(g, B, ks1, 2 * g->D_out))) return rc;
  if ((rc = reserve_decode(d, B, ks2, d->D_out))) return rc;
  if (!g_fused_swiglu && (rc = G->hidden.reserve((size_t)B * g->D_out * sizeof(float)))) return rc;
  DecodeWS ws;
  ws.phi = (_Float16*)g->Phi.p;
  ws.s = (float2*)g->S.p;
  ws.part = (float*)g->part.p;
  ws.phi2 = (_Float16*)d->Phi.p;
  ws.s2 = (float2*)d->S.p;
  ws.part2 = (float*)d->part.p;
  ws.cnt = (int*)g->cnt.p;
  ws.hidden = (float*)G->hidden.p;
  return gated_decode(G, X, x_dtype, ldx, Y, y_dtype, ldy, B, round16, ks1, ks2, ws, st);
}

// ---------------------------------------------------------------------------
// Workspace of kans_gated_forward_noalloc: one file-scope device array, held by
// every GPU the library runs on until the process ends.  Its first kScratchCnt
// bytes are the fused epilogue's arrival counters (zeroed once at set-up; every
// launch leaves them at zero again); one call's buffers are carved after them.
// Calls on one GPU share the array, so calls that overlap (other streams or
// threads) race.  In host code `scratch` names a host-side stand-in, never the
// device memory: the per-device address from hipGetSymbolAddress is used
// instead.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = size_t(64) << 20;
constexpr size_t kScratchCnt = size_t(256) << 10;  // 2048 row groups x kCntStride ints
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
std::map<int, char*> g_scratch;  // device -> address of that device's scratch (kans_mutex held)

__global__ void k_zero_words(unsigned* __restrict__ p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) p[i] = 0u;
}

// Carves 256-byte aligned buffers from the scratch after the counters.
struct ScratchCarve {
  char* base;
  size_t off = kScratchCnt, need = kScratchCnt;
  template <typename T>
  T* take(size_t bytes) {
    T* p = reinterpret_cast<T*>(base + off);
    off += (bytes + 255) / 256 * 256;
    need = off;
    return p;
  }
};

}  // namespace

// Set-up of the scratch on `device` (current): its address, and zeroed counters.
// Called once per device from the library's initialisation.
int kans_noalloc_setup(int device) {
  if (g_scratch.count(device)) return 0;
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr)
    return kans_fail(KANS_ERR_HIP, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
  hipStream_t st = kans_default_stream();
  hipLaunchKernelGGL(k_zero_words, dim3(64), dim3(256), 0, st, (unsigned*)ptr, (long)(kScratchCnt / 4));
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipStreamSynchronize(st));
  g_scratch[device] = (char*)ptr;
  return 0;
}

namespace {

// Host-pointer forward through grow-only device buffers and the library's
// pinned staging (stage_in / stage_out): X [B][D_in] is copied to rows of
// round_up(D_in, 8) elements (what the prefill kernel reads), the tail of
// each row zeroed.
template <typename Fwd>
int host_forward(DevBuf& hx, DevBuf& hy, const void* X, int x_dtype, int D_in, void* Y, int y_dtype, int D_out, int B,
                 Fwd&& fwd) {
  hipStream_t st = kans_default_stream();
  const long ldx = round_up(D_in, 8);
  const size_t xe = dt_bytes(x_dtype), ye = dt_bytes(y_dtype);
  const size_t xbytes = (size_t)B * ldx * xe, ybytes = (size_t)B * D_out * ye;
  int rc;
  if ((rc = hx.reserve(xbytes)) || (rc = hy.reserve(ybytes))) return rc;
  void* pin_in;
  void* pin_out;
  if ((rc = kans_pinned_stage(0, xbytes, &pin_in)) || (rc = kans_pinned_stage(1, ybytes, &pin_out))) return rc;
  if ((rc = stage_in(hx.p, X, (size_t)D_in * xe, (size_t)ldx * xe, B, pin_in, st))) return rc;
  if ((rc = fwd(hx.p, ldx, hy.p))) {
    (void)hipStreamSynchronize(st);  // the input DMAs read pin_in; finish them before another call reuses it
    return rc;
  }
  return stage_out(Y, hy.p, ybytes, pin_out, st);
}

// INT4 / INT8 layer from the reference arrays: decode records and prefill
// tiles (K in {1, 2, 4}) built from one upload of each array.
int create_affine(int bits, int D_in, int D_out, int K, int has_base, int has_bias, int group_size,
                  const void* qweight, const float* scales, const float* biases, const void* qweight_base,
                  const float* scales_base, const float* biases_base, const void* bias, int bias_dtype,
                  kans_qlayer** out) {
  const int quant = bits == 8 ? Q_INT8 : Q_INT4;
  if (!out || !qweight || !scales || !biases) return kans_fail(KANS_ERR_ARG, "null argument");
  if (has_base && (!qweight_base || !scales_base || !biases_base))
    return kans_fail(KANS_ERR_ARG, "has_base set but base arrays are null");
  int rc = validate_q(D_in, D_out, K, has_base, has_bias, group_size, quant);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(kans_mutex());
  if ((rc = kans_ensure_init())) return rc;
  hipStream_t st = kans_default_stream();
  auto* L = new kans_qlayer();
  L->quant = quant;
  L->D_in = D_in;
  L->D_out = D_out;
  L->K = K;
  L->has_base = has_base;
  L->has_bias = has_bias;
  L->group = group_size;
  layer_geometry(L);
  prefill_geometry(L);
  L->decode = true;
  auto fail = [&](int code) { delete L; return code; };
  if (L->decode && (rc = alloc_tiles(L))) return fail(rc);
  // one matrix (basis: D_out x D_in*K; base: D_out x D_in), rows padded to the group:
  // rows of pad / 2 (INT4) or pad (INT8) bytes, pad / 64 groups
  auto segment = [&](int seg, const void* q, const float* sc, const float* bi) -> int {
    const long kd = seg ? (long)D_in : (long)D_in * K;
    const long pad = (kd + group_size - 1) / group_size * group_size;
    const long gpr = pad / group_size;
    const long rowbytes = bits == 8 ? pad : pad / 2;
    DevBuf tq, ts, tb;
    int r;
    if ((r = upload_tmp(tq, q, (size_t)D_out * rowbytes, st))) return r;
    if ((r = upload_tmp(ts, sc, (size_t)D_out * gpr * 4, st))) return r;
    if ((r = upload_tmp(tb, bi, (size_t)D_out * gpr * 4, st))) return r;
    if (L->decode) {
      auto tile = quant == Q_INT8 ? qtile_int8 : qtile_int4;
      hipError_t e = tile((const unsigned char*)tq.p, (const float*)ts.p, (const float*)tb.p, D_out, rowbytes,
                          (int)gpr, L->nrb_pad, seg ? L->Cw : L->Cb, seg ? L->Cb : 0, L->C_tot, L->R.p, st);
      if (e != hipSuccess) return kans_fail(KANS_ERR_HIP, "INT%d re-tiling failed: %s", bits, hipGetErrorString(e));
    }
    if (L->prefill &&
        (r = build_ptiles(L, seg, tq.p, rowbytes, (const float*)ts.p, (const float*)tb.p, (int)gpr, st)))
      return r;
    HIP_TRY(hipStreamSynchronize(st));  // the temporaries die here
    return 0;
  };
  if ((rc = segment(0, qweight, scales, biases))) return fail(rc);
  if (has_base && (rc = segment(1, qweight_base, scales_base, biases_base))) return fail(rc);
  if ((rc = upload_bias(L, bias, bias_dtype))) return fail(rc);
  HIP_TRY(hipStreamSynchronize(st));
  *out = L;
  return 0;
}

// Mean ms per block forward, the calls cycling through the n blocks (n > 1: each
// call's weights were last read n - 1 calls earlier, so blocks whose weights
// together exceed the MALL are timed from HBM).  Lock held.
int time_blocks_locked(kans_gated* const* Gs, int n, const void* X, int x_dtype, void* Y, int y_dtype, int B,
                       int warmup, int iters, int use_graph, float* ms) {
  hipStream_t st = kans_default_stream();
  const int d = Gs[0]->gate->D_in;
  for (int b = 1; b < n; ++b)
    if (Gs[b]->gate->D_in != d || Gs[b]->down->D_out != Gs[0]->down->D_out)
      return kans_fail(KANS_ERR_ARG, "blocks of different shapes");
  std::vector<hipGraph_t> graphs(n, nullptr);
  std::vector<hipGraphExec_t> execs(n, nullptr);
  auto cleanup = [&]() {
    for (auto e : execs)
      if (e) (void)hipGraphExecDestroy(e);
    for (auto g : graphs)
      if (g) (void)hipGraphDestroy(g);
  };
  int rc = 0;
  for (int b = 0; b < n && !rc; ++b) {
    // one eager call sizes every workspace before any capture
    if ((rc = gated_forward_locked(Gs[b], X, x_dtype, d, Y, y_dtype, d, B, 1, st))) break;
    if (!use_graph) continue;
    hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
      rc = kans_fail(KANS_ERR_HIP, "hipStreamBeginCapture: %s", hipGetErrorString(e));
      break;
    }
    rc = gated_forward_locked(Gs[b], X, x_dtype, d, Y, y_dtype, d, B, 1, st);
    e = hipStreamEndCapture(st, &graphs[b]);
    if (!rc && e != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
    if (!rc && (e = hipGraphInstantiate(&execs[b], graphs[b], nullptr, nullptr, 0)) != hipSuccess)
      rc = kans_fail(KANS_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
  }
  auto run = [&](int i) -> int {
    const int b = i % n;
    if (use_graph) {
      HIP_TRY(hipGraphLaunch(execs[b], st));
      return 0;
    }
    return gated_forward_locked(Gs[b], X, x_dtype, d, Y, y_dtype, d, B, 1, st);
  };
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float t = 0.f;
  for (int i = 0; i < warmup && !rc; ++i) rc = run(i);
  if (!rc && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess))
    rc = kans_fail(KANS_ERR_HIP, "hipEventCreate failed");
  if (!rc && hipEventRecord(e0, st) != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "hipEventRecord failed");
  for (int i = 0; i < iters && !rc; ++i) rc = run(i);
  if (!rc && (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
              hipEventElapsedTime(&t, e0, e1) != hipSuccess))
    rc = kans_fail(KANS_ERR_HIP, "event timing failed");
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (rc) (void)hipStreamSynchronize(st);
  cleanup();
  if (!rc) *ms = t / iters;
  return rc;
}

// Mean ms per block forward of a decode step of n blocks captured as ONE HIP
// graph, as a model's step over its layers runs: block b reads the previous
// block's output (X -> Y -> X ..., so x_dtype == y_dtype), each block streams
// its own weights.  Lock held.
static int time_step_locked(kans_gated* const* Gs, int n, void* X, int dtype, void* Y, int B, int warmup, int iters,
                            float* ms) {
  hipStream_t st = kans_default_stream();
  const int d = Gs[0]->gate->D_in;
  for (int b = 0; b < n; ++b)
    if (Gs[b]->gate->D_in != d || Gs[b]->down->D_out != d)
      return kans_fail(KANS_ERR_ARG, "a decode step chains blocks of one width d -> d");
  auto step = [&]() -> int {
    for (int b = 0; b < n; ++b) {
      const void* in = (b & 1) ? Y : X;
      void* out = (b & 1) ? X : Y;
      int rc = gated_forward_locked(Gs[b], in, dtype, d, out, dtype, d, B, 1, st);
      if (rc) return rc;
    }
    return 0;
  };
  int rc = step();  // sizes every workspace before the capture
  if (rc) return rc;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  rc = step();
  hipError_t e = hipStreamEndCapture(st, &graph);
  if (!rc && e != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
  if (!rc && (e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0)) != hipSuccess)
    rc = kans_fail(KANS_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float t = 0.f;
  for (int i = 0; i < warmup && !rc; ++i)
    if (hipGraphLaunch(exec, st) != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "hipGraphLaunch failed");
  if (!rc && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess))
    rc = kans_fail(KANS_ERR_HIP, "hipEventCreate failed");
  if (!rc && hipEventRecord(e0, st) != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "hipEventRecord failed");
  for (int i = 0; i < iters && !rc; ++i)
    if (hipGraphLaunch(exec, st) != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "hipGraphLaunch failed");
  if (!rc && (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
              hipEventElapsedTime(&t, e0, e1) != hipSuccess))
    rc = kans_fail(KANS_ERR_HIP, "event timing failed");
  if (rc) (void)hipStreamSynchronize(st);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (exec) (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
  if (!rc) *ms = t / ((float)iters * n);
  return rc;
}

}  // namespace

extern "C" {

int kans_qlayer_create_int4(int D_in, int D_out, int K, int has_base, int has_bias, int group_size,
                            const void* qweight, const float* scales, const float* biases, const void* qweight_base,
                            const float* scales_base, const float* biases_base, const void* bias, int bias_dtype,
                            kans_qlayer** out) {
  return create_affine(4, D_in, D_out, K, has_base, has_bias, group_size, qweight, scales, biases, qweight_base,
                       scales_base, biases_base, bias, bias_dtype, out);
}

int kans_qlayer_create_int8(int D_in, int D_out, int K, int has_base, int has_bias, int group_size,
                            const void* qweight, const float* scales, const float* biases, const void* qweight_base,
                            const float* scales_base, const float* biases_base, const void* bias, int bias_dtype,
                            kans_qlayer** out) {
  return create_affine(8, D_in, D_out, K, has_base, has_bias, group_size, qweight, scales, biases, qweight_base,
                       scales_base, biases_base, bias, bias_dtype, out);
}

int kans_qlayer_create_ternary(int D_in, int D_out, int K, int has_base, int has_bias, int group_size,
                               const uint32_t* w_packed, const float* scales, const uint32_t* w_packed_base,
                               const float* scales_base, const void* bias, int bias_dtype, kans_qlayer** out) {
  if (!out || !w_packed || !scales) return kans_fail(KANS_ERR_ARG, "null argument");
  if (has_base && (!w_packed_base || !scales_base))
    return kans_fail(KANS_ERR_ARG, "has_base set but base arrays are null");
  int rc = validate_q(D_in, D_out, K, has_base, has_bias, group_size, Q_TERN);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(kans_mutex());
  if ((rc = kans_ensure_init())) return rc;
  hipStream_t st = kans_default_stream();
  auto* L = new kans_qlayer();
  L->quant = Q_TERN;
  L->D_in = D_in;
  L->D_out = D_out;
  L->K = K;
  L->has_base = has_base;
  L->has_bias = has_bias;
  L->group = group_size;
  layer_geometry(L);
  prefill_geometry(L);
  L->decode = true;
  auto fail = [&](int code) { delete L; return code; };
  if ((rc = alloc_tiles(L))) return fail(rc);
  // one matrix (basis: D_out x D_in*K; base: D_out x D_in): rows of ceil(kd / 16) words,
  // ceil(kd / 32) scales
  auto segment = [&](int seg, const uint32_t* wp, const float* sc) -> int {
    const long kd = seg ? (long)D_in : (long)D_in * K;
    const int wpr = (int)((kd + 15) / 16), gpr = (int)((kd + group_size - 1) / group_size);
    DevBuf tw, ts;
    int r;
    if ((r = upload_tmp(tw, wp, (size_t)D_out * wpr * 4, st))) return r;
    if ((r = upload_tmp(ts, sc, (size_t)D_out * gpr * 4, st))) return r;
    hipError_t e = qtile_tern((const unsigned*)tw.p, (const float*)ts.p, D_out, wpr, kd, gpr, L->nrb_pad,
                              seg ? L->Cw : L->Cb, seg ? L->Cb : 0, L->C_tot, L->R.p, st);
    if (e != hipSuccess) return kans_fail(KANS_ERR_HIP, "ternary re-tiling failed: %s", hipGetErrorString(e));
    if (L->prefill && (r = build_ptiles(L, seg, tw.p, wpr, (const float*)ts.p, nullptr, gpr, st))) return r;
    HIP_TRY(hipStreamSynchronize(st));  // the temporaries die here
    return 0;
  };
  if ((rc = segment(0, w_packed, scales))) return fail(rc);
  if (has_base && (rc = segment(1, w_packed_base, scales_base))) return fail(rc);
  if ((rc = upload_bias(L, bias, bias_dtype))) return fail(rc);
  HIP_TRY(hipStreamSynchronize(st));
  *out = L;
  return 0;
}

int kans_decode_set_weight_loads(int mode) {
  if (mode < 0 || mode > 2) return kans_fail(KANS_ERR_ARG, "weight-load mode must be 0, 1 or 2 (got %d)", mode);
  std::lock_guard<std::mutex> lk(kans_mutex());
  const int prev = g_weight_loads;
  g_weight_loads = mode;
  return prev;
}

int kans_prefill_set_block_pairs(int on) {
  if (on != 0 && on != 1) return kans_fail(KANS_ERR_ARG, "block pairs must be 0 or 1 (got %d)", on);
  std::lock_guard<std::mutex> lk(kans_mutex());
  const int prev = g_qp_block_pairs;
  g_qp_block_pairs = on;
  return prev;
}

int kans_gated_set_fused_swiglu(int on) {
  std::lock_guard<std::mutex> lk(kans_mutex());
  const int prev = g_fused_swiglu ? 1 : 0;
  g_fused_swiglu = on != 0;
  return prev;
}

int kans_decode_set_pre_basis(int on) {
  std::lock_guard<std::mutex> lk(kans_mutex());
  if (on < 0 || on > 2) return kans_fail(KANS_ERR_ARG, "pre-basis mode %d not in 0..2", on);
  const int prev = g_pre_basis;
  g_pre_basis = on;
  return prev;
}

int kans_qlayer_destroy(kans_qlayer* L) {
  if (!L) return 0;
  std::lock_guard<std::mutex> lk(kans_mutex());
  if (kans_default_stream()) (void)hipStreamSynchronize(kans_default_stream());
  delete L;
  return 0;
}

int kans_qlayer_forward(kans_qlayer* L, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy, int B,
                        void* stream) {
  if (!L) return kans_fail(KANS_ERR_ARG, "null layer");
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  hipStream_t st = stream ? (hipStream_t)stream : kans_default_stream();
  return qlayer_forward_locked(L, X, x_dtype, ldx, Y, y_dtype, ldy, B, st);
}

int kans_qlayer_forward_host(kans_qlayer* L, const void* X, int x_dtype, void* Y, int y_dtype, int B) {
  if (!L || (B > 0 && (!X || !Y))) return kans_fail(KANS_ERR_ARG, "null argument");
  if (B < 0) return kans_fail(KANS_ERR_ARG, "B=%d < 0", B);
  if (x_dtype < DT_F32 || x_dtype > DT_BF16 || y_dtype < DT_F32 || y_dtype > DT_BF16)
    return kans_fail(KANS_ERR_ARG, "bad x / y dtype");
  if (B == 0) return 0;
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  hipStream_t st = kans_default_stream();
  return host_forward(L->hx, L->hy, X, x_dtype, L->D_in, Y, y_dtype, L->D_out, B, [&](void* dx, long ldx, void* dy) {
    return qlayer_forward_locked(L, dx, x_dtype, ldx, dy, y_dtype, L->D_out, B, st);
  });
}

int kans_qlayer_set_rbf(kans_qlayer* L, const float* centers, float inv_denominator) {
  if (!L || !centers) return kans_fail(KANS_ERR_ARG, "null argument");
  std::lock_guard<std::mutex> lk(kans_mutex());
  BasisParams bp{};
  bp.K = L->K;
  if (!kans_set_rbf_params(bp, centers, inv_denominator))
    return kans_fail(KANS_ERR_ARG, "RBF inv_denominator must be finite and >= 0");
  L->bp = bp;
  L->basis = BASIS_RBF;
  return 0;
}

int kans_qlayer_set_bspline(kans_qlayer* L, int grid_size, float grid_min, float inv_h) {
  if (!L) return kans_fail(KANS_ERR_ARG, "null layer");
  if (grid_size <= 0 || grid_size + 3 != L->K)
    return kans_fail(KANS_ERR_ARG, "grid_size=%d inconsistent with K=%d (K = G + 3)", grid_size, L->K);
  std::lock_guard<std::mutex> lk(kans_mutex());
  BasisParams bp{};
  bp.K = L->K;
  bp.grid_size = grid_size;
  bp.grid_min = grid_min;
  bp.inv_h = inv_h;
  L->bp = bp;
  L->basis = BASIS_BSPLINE;
  return 0;
}

int kans_qlayer_fused(const kans_qlayer* L, int B) {
  if (!L) return 0;
  if (B <= 0) return 1;
  if (B <= kMaxDecodeB && L->decode) return 1;
  return prefill_ok(L) ? 1 : 0;
}

int kans_gated_create(kans_qlayer* gate, kans_qlayer* up, kans_qlayer* down, kans_gated** out) {
  if (!gate || !up || !down || !out) return kans_fail(KANS_ERR_ARG, "null argument");
  if (gate->basis != BASIS_CHEBY || up->basis != BASIS_CHEBY || down->basis != BASIS_CHEBY)
    return kans_fail(KANS_ERR_ARG, "the GatedKAN block takes Chebyshev layers (gated_kan.py:36-84)");
  if (gate->quant != up->quant || gate->quant != down->quant)
    return kans_fail(KANS_ERR_ARG, "gate, up and down must share one quantization format");
  if (gate->D_in != up->D_in || gate->D_out != up->D_out || gate->K != up->K || gate->has_base != up->has_base ||
      down->D_in != gate->D_out || down->D_out != gate->D_in)
    return kans_fail(KANS_ERR_ARG, "shape mismatch: gate/up %dx%d, down %dx%d", gate->D_in, gate->D_out, down->D_in,
                     down->D_out);
  auto* G = new kans_gated();
  G->gate = gate;
  G->up = up;
  G->down = down;
  *out = G;
  return 0;
}

int kans_gated_destroy(kans_gated* G) {
  if (!G) return 0;
  std::lock_guard<std::mutex> lk(kans_mutex());
  if (kans_default_stream()) (void)hipStreamSynchronize(kans_default_stream());
  delete G;
  return 0;
}

int kans_gated_forward(kans_gated* G, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy, int B,
                       int round16, void* stream) {
  if (!G) return kans_fail(KANS_ERR_ARG, "null block");
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  hipStream_t st = stream ? (hipStream_t)stream : kans_default_stream();
  return gated_forward_locked(G, X, x_dtype, ldx, Y, y_dtype, ldy, B, round16, st);
}

int kans_gated_forward_host(kans_gated* G, const void* X, int x_dtype, void* Y, int y_dtype, int B, int round16) {
  if (!G || (B > 0 && (!X || !Y))) return kans_fail(KANS_ERR_ARG, "null argument");
  if (B < 0) return kans_fail(KANS_ERR_ARG, "B=%d < 0", B);
  if (x_dtype < DT_F32 || x_dtype > DT_BF16 || y_dtype < DT_F32 || y_dtype > DT_BF16)
    return kans_fail(KANS_ERR_ARG, "bad x / y dtype");
  if (B == 0) return 0;
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  hipStream_t st = kans_default_stream();
  const int d = G->gate->D_in;
  return host_forward(G->hx, G->hy, X, x_dtype, d, Y, y_dtype, d, B, [&](void* dx, long ldx, void* dy) {
    return gated_forward_locked(G, dx, x_dtype, ldx, dy, y_dtype, d, B, round16, st);
  });
}

// As kans_gated_forward, with every workspace carved from the library's
// per-GPU scratch array (no allocation on this path).
int kans_gated_forward_noalloc(kans_gated* G, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy,
                               int B, int round16, void* stream) {
  if (!G) return kans_fail(KANS_ERR_ARG, "null block");
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  int dev = -1;
  HIP_TRY(hipGetDevice(&dev));
  auto it = g_scratch.find(dev);
  if (it == g_scratch.end()) return kans_fail(KANS_ERR_STATE, "no scratch set up on device %d", dev);
  hipStream_t st = stream ? (hipStream_t)stream : kans_default_stream();
  kans_qlayer *g = G->gate, *d = G->down;
  if ((rc = check_y(Y, y_dtype, ldy, d->D_out))) return rc;
  if (B < 0) return kans_fail(KANS_ERR_ARG, "B=%d < 0", B);
  if (B == 0) return 0;
  ScratchCarve sc{it->second};
  auto too_big = [&](size_t need) {
    return kans_fail(KANS_ERR_ARG,
                     "kans_gated_forward_noalloc: B=%d needs %zu bytes of workspace, above the %zu-byte scratch "
                     "(use kans_gated_forward)", B, need, kScratchBytes);
  };
  if (B > kMaxDecodeB || !g->decode) {
    GatedPrefill GP;
    if ((rc = plan_gated_prefill(G, X, x_dtype, ldx, Y, y_dtype, ldy, B, round16, GP))) return rc;
    void* hidden = sc.take<char>(GP.hidden_bytes);
    float* part = GP.part_bytes ? sc.take<float>(GP.part_bytes) : nullptr;
    if (sc.need > kScratchBytes) return too_big(sc.need);
    return run_gated_prefill(GP, hidden, part, st);
  }
  if ((rc = check_x(X, x_dtype, ldx, g->D_in, B))) return rc;
  if ((size_t)(g->nrb_pad / g->nw) * kCntStride * sizeof(int) > kScratchCnt)
    return kans_fail(KANS_ERR_ARG, "kans_gated_forward_noalloc: %d gate row groups exceed the scratch counters",
                     g->nrb_pad / g->nw);
  int ks1, ks2;
  gated_ksplits(G, B, &ks1, &ks2);
  DecodeWS ws;
  ws.cnt = (int*)it->second;
  ws.phi = sc.take<_Float16>(phi_bytes(g, B));
  ws.s = sc.take<float2>(s_bytes(g, B));
  ws.part = sc.take<float>(part_bytes(B, ks1, 2 * g->D_out));
  ws.phi2 = sc.take<_Float16>(phi_bytes(d, B));
  ws.s2 = sc.take<float2>(s_bytes(d, B));
  ws.part2 = sc.take<float>(part_bytes(B, ks2, d->D_out));
  if (!g_fused_swiglu) ws.hidden = sc.take<float>((size_t)B * g->D_out * sizeof(float));
  if (sc.need > kScratchBytes) return too_big(sc.need);
  return gated_decode(G, X, x_dtype, ldx, Y, y_dtype, ldy, B, round16, ks1, ks2, ws, st);
}

// Mean time of one block forward on device-resident X / Y; use_graph replays
// the six launches as one captured HIP graph.
int kans_gated_time(kans_gated* G, const void* X, int x_dtype, void* Y, int y_dtype, int B, int warmup, int iters,
                    int use_graph, float* ms) {
  if (!G || !X || !Y || !ms || iters <= 0) return kans_fail(KANS_ERR_ARG, "bad argument");
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  return time_blocks_locked(&G, 1, X, x_dtype, Y, y_dtype, B, warmup, iters, use_graph, ms);
}

int kans_gated_time_step(kans_gated* const* blocks, int n, void* X, void* Y, int dtype, int B, int warmup, int iters,
                         float* ms) {
  if (!blocks || n <= 0 || !X || !Y || !ms || iters <= 0 || B <= 0) return kans_fail(KANS_ERR_ARG, "bad argument");
  for (int b = 0; b < n; ++b)
    if (!blocks[b]) return kans_fail(KANS_ERR_ARG, "null block");
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  return time_step_locked(blocks, n, X, dtype, Y, B, warmup, iters, ms);
}

int kans_gated_time_rotate(kans_gated* const* blocks, int n, const void* X, int x_dtype, void* Y, int y_dtype, int B,
                           int warmup, int iters, float* ms) {
  if (!blocks || n <= 0 || !X || !Y || !ms || iters <= 0) return kans_fail(KANS_ERR_ARG, "bad argument");
  for (int b = 0; b < n; ++b)
    if (!blocks[b]) return kans_fail(KANS_ERR_ARG, "null block");
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  return time_blocks_locked(blocks, n, X, x_dtype, Y, y_dtype, B, warmup, iters, 1, ms);
}

// Packed bytes the decode path streams per block forward (weights + group
// parameters as stored by the reference formats, activations in, result out):
// the algorithmic traffic used for the HBM roofline.
long long kans_gated_stream_bytes(const kans_gated* G, int B) {
  if (!G) return -1;
  long long total = 0;
  for (const kans_qlayer* L : {G->gate, G->up, G->down}) {
    const long kb = (long)L->D_in * L->K;
    for (int part = 0; part < 1 + L->has_base; ++part) {
      const long kdim = part == 0 ? kb : L->D_in;
      if (L->quant == Q_INT4 || L->quant == Q_INT8) {
        const long pad = (kdim + L->group - 1) / L->group * L->group;
        total += (long long)L->D_out * ((L->quant == Q_INT8 ? pad : pad / 2) + (pad / L->group) * 8);
      } else {
        total += (long long)L->D_out * (((kdim + 15) / 16) * 4 + ((kdim + L->group - 1) / L->group) * 4);
      }
    }
  }
  total += (long long)B * G->gate->D_in * 2 * 2;  // x in, y out (fp16)
  return total;
}

// Reference fused ternary forward (metal_kan_bridge.mm:4684-4733): fp32 X, no
// base branch, ternary W (D_out x D_in*degree), optional fp32 bias.  Computed
// in fp32 on the exact dequantized weights (the same arithmetic contract as
// the reference kernel), so results match the fp32 oracle to 1e-4.  The codes
// are dequantized into a device buffer that the fused fp32 kernel's weight
// re-tiling reads directly: the fp32 weights never leave the device.
int metal_kan_forward_ternary_cheby(const float* X, const uint32_t* W_packed, const float* scales, const float* bias,
                                    float* Y, int B, int D_in, int D_out, int degree, int group_size, int has_bias) {
  if (!X || !W_packed || !scales || !Y || B <= 0 || D_in <= 0 || D_out <= 0 || degree <= 0 || group_size <= 0)
    return kans_fail(KANS_ERR_ARG, "bad argument");
  if (degree > kMaxK) return kans_fail(KANS_ERR_ARG, "degree %d > %d", degree, kMaxK);
  if (has_bias && !bias) return kans_fail(KANS_ERR_ARG, "has_bias=1 but bias is null");
  std::lock_guard<std::mutex> lk(kans_mutex());
  int rc = kans_ensure_init();
  if (rc) return rc;
  hipStream_t st = kans_default_stream();
  const long kd = (long)D_in * degree;
  const size_t pbytes = (size_t)D_out * ((kd + 15) / 16) * 4, sbytes = (size_t)D_out * ((kd + group_size - 1) / group_size) * 4;
  DevBuf dp, ds, dw, db;
  if ((rc = upload_tmp(dp, W_packed, pbytes, st)) || (rc = upload_tmp(ds, scales, sbytes, st)) ||
      (rc = dw.reserve((size_t)D_out * kd * 4)))
    return rc;
  if (has_bias && (rc = upload_tmp(db, bias, (size_t)D_out * 4, st))) return rc;
  if ((rc = dequant_ternary_device((const uint32_t*)dp.p, (const float*)ds.p, (float*)dw.p, D_out, (int)kd,
                                   group_size, st)))
    return rc;
  // the weight upload synchronises the stream after re-tiling, before these buffers are released
  return kans_ref_cheby_forward_devw_locked(X, (const float*)dw.p, has_bias ? (const float*)db.p : nullptr, Y, B,
                                            D_in, D_out, degree, has_bias ? 1 : 0);
}

}  // extern "C"
