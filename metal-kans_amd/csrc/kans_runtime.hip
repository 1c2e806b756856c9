// Host runtime and C-ABI of the MI355X fused KAN library (libkans_hip.so).
//
// Replaces the reference's Objective-C++ bridge for the hot path
// (metal_kans/kernels/metal_kan_bridge.mm): device/queue setup (:289-404), the
// zero-copy host buffer cache (:409-441), the fp32/fp16 forwards
// (:443-625,1069-1164,1890-2151), the chain pipeline (:1168-1248), the async
// flag (:84-97,275-287) and the benchmark helpers (:1250-1371).
//
// Design (MI355X, discrete HBM):
//   * one HIP device, one non-blocking stream at default priority;
//   * a kans_layer owns its weights in HBM, re-tiled once on upload for the
//     fused kernel; the reference-named entry points keep their semantics (the
//     host arrays are read on every call) by uploading through a layer cache;
//   * host arrays move through pinned staging buffers with hipMemcpyAsync;
//   * async mode defers the copy of results into the caller's arrays to
//     metal_kan_sync();
//   * every entry point validates its arguments before any HIP call and
//     returns 0 or a negative code; kans_last_error() describes the failure.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <cmath>
#include <string>
#include <tuple>
#include <vector>
#include <chrono>

#include "kans_common.h"
#include "kans_api_internal.h"

using namespace kans;

namespace kans {
hipError_t launch_dense(const DenseLaunch& L, hipStream_t st);
bool dense_config_supported(int wm, int nb);
bool block_wave_groups_ok(int wm, int nb, int ks);
int block_waves(bool half, int basis, int wm, int nb, int KP);
hipError_t launch_repack(int src_dtype, int dtype, const void* W, const void* Wb, void* Wt, int D_in, int D_out,
                         int K, int has_base, int nfb, int nob_pad, hipStream_t st);
hipError_t launch_convert(int src_dtype, int dtype, const void* src, void* dst, long n, hipStream_t st);
}  // namespace kans

// ---------------------------------------------------------------------------
// Errors
// ---------------------------------------------------------------------------
static thread_local std::string g_err;

int kans_fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// ---------------------------------------------------------------------------
// Device state
// ---------------------------------------------------------------------------
static std::mutex g_mu;            // serialises the library (the reference is single-threaded too)
static bool g_ready = false;
static int g_device = -1;
static hipStream_t g_stream = nullptr;
// copy streams and second compute stream of the chunked host forward (layer_forward_host_chunked)
static hipStream_t g_copy_in = nullptr, g_copy_out = nullptr, g_compute2 = nullptr;
static thread_local int g_async = 0;  // reference: thread_local g_async_mode

struct Pending {  // a deferred device->host result copy (async mode); dst null: just free
  void* pinned;
  void* dst;
  size_t bytes;
};
static std::vector<Pending> g_pending;

// grow-only pinned staging buffers (synchronous mode)
static Pinned g_pin_in, g_pin_out;

static int ensure_init() {
  if (g_ready) return 0;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0)
    return kans_fail(KANS_ERR_NODEV, "no HIP device visible (hipGetDeviceCount: %s, count=%d)",
                     hipGetErrorString(e), n);
  HIP_TRY(hipGetDevice(&g_device));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, g_device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return kans_fail(KANS_ERR_NODEV, "device %d is %s; this library is built for gfx950 only", g_device,
                     prop.gcnArchName);
  HIP_TRY(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  HIP_TRY(hipStreamCreateWithFlags(&g_copy_in, hipStreamNonBlocking));
  HIP_TRY(hipStreamCreateWithFlags(&g_copy_out, hipStreamNonBlocking));
  HIP_TRY(hipStreamCreateWithFlags(&g_compute2, hipStreamNonBlocking));
  int rc = kans_noalloc_setup(g_device);
  if (rc) return rc;
  g_ready = true;
  return 0;
}

hipStream_t kans_default_stream() { return g_stream; }

std::mutex& kans_mutex() { return g_mu; }
int kans_ensure_init() { return ensure_init(); }
int kans_pinned_stage(int which, size_t bytes, void** p) {
  Pinned& b = which ? g_pin_out : g_pin_in;
  int rc = pinned_reserve(b, bytes);
  if (rc) return rc;
  *p = b.p;
  return 0;
}

static size_t dtype_size(int dt) { return dt == DT_F32 ? 4 : 2; }

// ---------------------------------------------------------------------------
// Layer
// ---------------------------------------------------------------------------
struct kans_layer {
  int basis, dtype, D_in, D_out, K, has_base, has_bias;
  int D_in8, nfb, nob_pad;
  BasisParams bp{};
  DevBuf Wt, bias_d, part, x_d, y_d, raw_w, raw_wb;
  bool have_weights = false;
  int forced_wm = 0, forced_nb = 0, forced_splits = 0;  // tuning overrides (0 = heuristic)
  int forced_ks = 0;  // wave groups per workgroup override (0 = heuristic)
  int block_pairs = 1;  // block kernels: two feature blocks per LDS stage when they fit
  unsigned gen = 0;  // bumped whenever a buffer captured by a graph may have moved
};

// Scaled-centre table of the RBF basis: phi_k = exp2(-(s*x - s*c_k)^2) with
// s = sqrt(-neg_l), the form BasisGen<BASIS_RBF> evaluates.
// Reference layers derive inv_denominator = 1 / (2 h^2) >= 0 (fast_kan.py:42);
// a negative one (a growing "Gaussian") has no real scale s and is rejected.
static bool rbf_inv_den_ok(float inv_den) { return inv_den >= 0.0f && std::isfinite(inv_den); }

static void set_rbf_table(BasisParams& bp) {
  const double sq = bp.neg_l < 0.0f ? std::sqrt(-(double)bp.neg_l) : 0.0;
  bp.rbf_s = (float)sq;
  for (int k = 0; k < bp.K; ++k) bp.rbf_sc[k] = (float)(sq * (double)bp.centers[k]);
  // Recurrence (BASIS_RBF_REC, 16-bit block kernel only) when the centres are
  // uniform to 1e-3 of their spacing h and the scaled span is at most
  // kRbfRecSpan; otherwise exp2 per value.  The tolerance admits a uniform grid
  // stored in fp16 (FastKAN.half() rounds the centres: 2.3e-4 h at config 3);
  // moving a centre by dc changes phi by at most sqrt(2 inv_den / e) |dc|
  // (e = 2.718...), i.e. 6e-4 for the reference's inv_den = 1 / (2 h^2) and
  // |dc| = 1e-3 h: the size of the fp16 rounding of phi itself.
  bp.rbf_rec = 0;
  const int K = bp.K;
  if (K < 2 || !(sq > 0.0)) return;
  const double c0 = sq * (double)bp.centers[0];
  const double d = (sq * (double)bp.centers[K - 1] - c0) / (K - 1);
  if (!(d > 0.0) || !std::isfinite(d) || (K - 1) * d > (double)kRbfRecSpan) return;
  for (int k = 0; k < K; ++k)
    if (std::fabs(sq * (double)bp.centers[k] - (c0 + k * d)) > 1e-3 * d) return;
  bp.rec_lo = -kRbfRecPad;
  bp.rec_hi = (float)((K - 1) * d + (double)kRbfRecPad);
  bp.rec_2d = (float)(2.0 * d);
  bp.rec_c = (float)(-d * d);
  bp.rec_q = (float)std::exp2(-2.0 * d * d);
  bp.rbf_rec = 1;
}

// RBF basis parameters of K centres and 1/(2h^2) (for the quantized layers, kans_qruntime.hip);
// false for an inv_denominator the layers refuse.
bool kans::kans_set_rbf_params(BasisParams& bp, const float* centers, float inv_den) {
  if (!rbf_inv_den_ok(inv_den)) return false;
  for (int k = 0; k < bp.K; ++k) bp.centers[k] = centers[k];
  bp.have_centers = 1;
  bp.neg_l = -inv_den * kLog2e;
  set_rbf_table(bp);
  return true;
}

static int validate_dims(int basis, int dtype, int D_in, int D_out, int K, int has_base, int has_bias) {
  if (basis < 0 || basis > 2) return kans_fail(KANS_ERR_ARG, "unknown basis %d", basis);
  if (dtype < 0 || dtype > 2) return kans_fail(KANS_ERR_ARG, "unknown dtype %d", dtype);
  if (D_in <= 0 || D_out <= 0) return kans_fail(KANS_ERR_ARG, "bad dims D_in=%d D_out=%d", D_in, D_out);
  if (K <= 0 || K > kMaxK) return kans_fail(KANS_ERR_ARG, "K=%d outside [1, %d]", K, kMaxK);
  if ((has_base != 0 && has_base != 1) || (has_bias != 0 && has_bias != 1))
    return kans_fail(KANS_ERR_ARG, "has_base/has_bias must be 0 or 1");
  return 0;
}

extern "C" {

const char* kans_last_error(void) { return g_err.c_str(); }

int kans_layer_create(int basis, int dtype, int D_in, int D_out, int K, int has_base, int has_bias,
                      kans_layer** out) {
  if (!out) return kans_fail(KANS_ERR_ARG, "null out pointer");
  int rc = validate_dims(basis, dtype, D_in, D_out, K, has_base, has_bias);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  if ((rc = ensure_init())) return rc;
  auto* L = new kans_layer();
  L->basis = basis;
  L->dtype = dtype;
  L->D_in = D_in;
  L->D_out = D_out;
  L->K = K;
  L->has_base = has_base;
  L->has_bias = has_bias;
  L->D_in8 = round_up(D_in, 8);
  L->nfb = (D_in + 15) / 16;
  L->nob_pad = round_up((D_out + 31) / 32, kObPad);
  L->bp.K = K;
  *out = L;
  return 0;
}

int kans_layer_destroy(kans_layer* L) {
  if (!L) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ready) (void)hipStreamSynchronize(g_stream);
  delete L;
  return 0;
}

int kans_layer_set_rbf(kans_layer* L, const float* centers, float inv_den) {
  if (!L || !centers) return kans_fail(KANS_ERR_ARG, "null argument");
  if (L->basis != BASIS_RBF) return kans_fail(KANS_ERR_ARG, "layer basis is not RBF");
  if (!rbf_inv_den_ok(inv_den)) return kans_fail(KANS_ERR_ARG, "RBF inv_denominator must be finite and >= 0");
  std::lock_guard<std::mutex> lk(g_mu);
  for (int k = 0; k < L->K; ++k) L->bp.centers[k] = centers[k];
  L->bp.have_centers = 1;
  L->bp.neg_l = -inv_den * kLog2e;
  set_rbf_table(L->bp);
  ++L->gen;  // the kernel arguments captured by a chain graph change
  return 0;
}

int kans_layer_set_bspline(kans_layer* L, int grid_size, float grid_min, float inv_h) {
  if (!L) return kans_fail(KANS_ERR_ARG, "null layer");
  if (L->basis != BASIS_BSPLINE) return kans_fail(KANS_ERR_ARG, "layer basis is not B-spline");
  if (grid_size <= 0 || grid_size + 3 != L->K)
    return kans_fail(KANS_ERR_ARG, "grid_size=%d inconsistent with K=%d (K = G + 3)", grid_size, L->K);
  L->bp.grid_size = grid_size;
  L->bp.grid_min = grid_min;
  L->bp.inv_h = inv_h;
  ++L->gen;  // basis parameters are baked into captured kernel arguments
  return 0;
}

int kans_layer_set_tiling(kans_layer* L, int wm, int nb, int splits) {
  if (!L) return kans_fail(KANS_ERR_ARG, "null layer");
  if (wm != 0 && wm != 32 && wm != 64) return kans_fail(KANS_ERR_ARG, "wm must be 0, 32 or 64");
  if ((wm == 0) != (nb == 0)) return kans_fail(KANS_ERR_ARG, "wm and nb must both be 0 or both set");
  if (wm != 0 && !dense_config_supported(wm, nb))
    return kans_fail(KANS_ERR_ARG, "tile (wm=%d, nb=%d) not instantiated; use (64,4) (32,8) (32,4) (32,1)", wm, nb);
  if (splits < 0) return kans_fail(KANS_ERR_ARG, "splits must be >= 0");
  L->forced_wm = wm;
  L->forced_nb = nb;
  L->forced_splits = splits;
  ++L->gen;
  return 0;
}

int kans_layer_set_wave_groups(kans_layer* L, int groups) {
  if (!L) return kans_fail(KANS_ERR_ARG, "null layer");
  if (groups != 0 && groups != 1 && groups != 2 && groups != 4)
    return kans_fail(KANS_ERR_ARG, "wave groups must be 0 (automatic), 1, 2 or 4");
  L->forced_ks = groups;
  ++L->gen;
  return 0;
}

int kans_layer_set_block_pairs(kans_layer* L, int on) {
  if (!L) return kans_fail(KANS_ERR_ARG, "null layer");
  if (on != 0 && on != 1) return kans_fail(KANS_ERR_ARG, "block pairs must be 0 or 1");
  L->block_pairs = on;
  ++L->gen;
  return 0;
}

// Upload weights (host or device memory) whose element type is src_dtype (the
// layer dtype, or fp32 for a converting upload).  W: [D_out][D_in*K];
// W_base: [D_out][D_in] (ignored unless has_base); bias: [D_out] (ignored
// unless has_bias).  Re-tiles W/W_base into the fused kernel's layout.
static int layer_upload_locked(kans_layer* L, const void* W, const void* Wb, const void* bias, bool device_src,
                               int src_dtype) {
  const size_t es = dtype_size(src_dtype);
  const size_t wbytes = (size_t)L->D_out * L->D_in * L->K * es;
  const size_t wbbytes = (size_t)L->D_out * L->D_in * es;
  const int KP = L->K + L->has_base;
  const size_t tbytes = (size_t)L->nfb * KP * L->nob_pad * 64 * 16 * (L->dtype == DT_F32 ? 2 : 1);
  int rc;
  void* old_wt = L->Wt.p;
  void* old_bias = L->bias_d.p;
  if ((rc = L->Wt.reserve(tbytes))) return rc;
  const void* w_src = W;
  const void* wb_src = Wb;
  const void* b_src = bias;
  if (!device_src) {
    if ((rc = L->raw_w.reserve(wbytes + (L->has_bias ? (size_t)L->D_out * es : 0)))) return rc;
    HIP_TRY(hipMemcpyAsync(L->raw_w.p, W, wbytes, hipMemcpyHostToDevice, g_stream));
    w_src = L->raw_w.p;
    if (L->has_bias) {
      HIP_TRY(hipMemcpyAsync((char*)L->raw_w.p + wbytes, bias, (size_t)L->D_out * es, hipMemcpyHostToDevice,
                             g_stream));
      b_src = (char*)L->raw_w.p + wbytes;
    }
    if (L->has_base) {
      if ((rc = L->raw_wb.reserve(wbbytes))) return rc;
      HIP_TRY(hipMemcpyAsync(L->raw_wb.p, Wb, wbbytes, hipMemcpyHostToDevice, g_stream));
      wb_src = L->raw_wb.p;
    }
  }
  HIP_TRY(launch_repack(src_dtype, L->dtype, w_src, L->has_base ? wb_src : nullptr, L->Wt.p, L->D_in, L->D_out,
                        L->K, L->has_base, L->nfb, L->nob_pad, g_stream));
  if (L->has_bias) {
    const size_t bbytes = (size_t)L->D_out * dtype_size(L->dtype);
    if ((rc = L->bias_d.reserve(bbytes))) return rc;
    if (src_dtype == L->dtype) {
      HIP_TRY(hipMemcpyAsync(L->bias_d.p, b_src, bbytes, hipMemcpyDeviceToDevice, g_stream));
    } else {
      HIP_TRY(launch_convert(src_dtype, L->dtype, b_src, L->bias_d.p, L->D_out, g_stream));
    }
  }
  HIP_TRY(hipStreamSynchronize(g_stream));
  if (L->Wt.p != old_wt || L->bias_d.p != old_bias) ++L->gen;
  L->have_weights = true;
  return 0;
}

int kans_layer_load_weights(kans_layer* L, const void* W, const void* W_base, const void* bias) {
  if (!L || !W) return kans_fail(KANS_ERR_ARG, "null layer or W");
  if (L->has_base && !W_base) return kans_fail(KANS_ERR_ARG, "has_base=1 but W_base is null");
  if (L->has_bias && !bias) return kans_fail(KANS_ERR_ARG, "has_bias=1 but bias is null");
  std::lock_guard<std::mutex> lk(g_mu);
  return layer_upload_locked(L, W, W_base, bias, false, L->dtype);
}

int kans_layer_load_weights_f32(kans_layer* L, const float* W, const float* W_base, const float* bias) {
  if (!L || !W) return kans_fail(KANS_ERR_ARG, "null layer or W");
  if (L->has_base && !W_base) return kans_fail(KANS_ERR_ARG, "has_base=1 but W_base is null");
  if (L->has_bias && !bias) return kans_fail(KANS_ERR_ARG, "has_bias=1 but bias is null");
  std::lock_guard<std::mutex> lk(g_mu);
  return layer_upload_locked(L, W, W_base, bias, false, DT_F32);
}

int kans_layer_load_weights_device(kans_layer* L, const void* W, const void* W_base, const void* bias) {
  if (!L || !W) return kans_fail(KANS_ERR_ARG, "null layer or W");
  if (L->has_base && !W_base) return kans_fail(KANS_ERR_ARG, "has_base=1 but W_base is null");
  if (L->has_bias && !bias) return kans_fail(KANS_ERR_ARG, "has_bias=1 but bias is null");
  std::lock_guard<std::mutex> lk(g_mu);
  return layer_upload_locked(L, W, W_base, bias, true, L->dtype);
}

}  // extern "C"

// Tile configuration.  Preference orders come from MI355X timings at
// 16384 x 1024 -> 1024 (16-bit) and 8192 x 1024 -> {1024, 4096} (fp32):
//   16-bit, every basis (32,8) -- the 8-wave block kernel: 8 basis values per
//                                lane feed 8 MFMAs;
//   fp32 Chebyshev / RBF (32,4); fp32 B-spline (32,8).
// 1. The first shape in that order whose tiles alone fill every CU's resident
//    workgroup slots (256 for the 8-wave block kernel, 512 otherwise).
// 2. Else the first of (32,4), (32,8), (64,4), (32,1) that fills half of them
//    with a feature split of at most nfb / 8 (>= 8 feature blocks per split):
//    measured on the config-2 chain's layers (4096 x 784 -> 256 best at
//    (32,4) x 4 splits, 4096 x 256 -> 256 at (32,1) unsplit).
// 3. Else the shape with the most tiles, split towards 512 workgroups, at most
//    nfb / 2 ways on the block kernel (4096 x 256 -> 10: (32,1) x 8) and nfb
//    ways on the per-slot kernel.
static void choose_tiling(const kans_layer* L, int B, int* wm, int* nb, int* splits) {
  static const int pref_n8[4][2] = {{32, 8}, {64, 4}, {32, 4}, {32, 1}};
  static const int pref_n4[4][2] = {{32, 4}, {64, 4}, {32, 8}, {32, 1}};
  static const int pref_small[4][2] = {{32, 4}, {32, 8}, {64, 4}, {32, 1}};
  const bool f32 = L->dtype == DT_F32;
  const int(*cand)[2] = (f32 && L->basis != BASIS_BSPLINE) ? pref_n4 : pref_n8;
  const int nob = (L->D_out + 31) / 32;
  const int KP = L->K + L->has_base;
  // workgroups of shape (ww, nn): the 8-wave block kernel's tile is 8 row blocks tall
  auto waves_of = [&](int ww, int nn) { return block_waves(!f32, L->basis, ww, nn, KP) == 8 ? 8 : 4; };
  auto wgs = [&](int ww, int nn) {
    const int rows = waves_of(ww, nn) * ww;
    return ((B + rows - 1) / rows) * ((nob + nn - 1) / nn);
  };
  auto slots = [&](int ww, int nn) { return waves_of(ww, nn) == 8 ? 256 : 512; };
  auto mostly_padding = [&](int nn) {
    const int padded = ((nob + nn - 1) / nn) * nn;
    return nn > 1 && 2 * nob < padded;  // over half of the N-tile would be padding
  };
  int bw = 0, bn = 0, s = 1;
  for (int i = 0; i < 4 && !bw; ++i) {
    const int* c = cand[i];
    if (!mostly_padding(c[1]) && wgs(c[0], c[1]) >= slots(c[0], c[1])) { bw = c[0]; bn = c[1]; }
  }
  const int smax = std::max(1, L->nfb / 8);
  for (int i = 0; i < 4 && !bw; ++i) {
    const int* c = pref_small[i];
    if (mostly_padding(c[1])) continue;
    const int t = wgs(c[0], c[1]), need = slots(c[0], c[1]) / 2;
    const int sc = std::min(smax, (need + t - 1) / t);
    if ((long)t * sc >= need) { bw = c[0]; bn = c[1]; s = sc; }
  }
  if (!bw) {
    bw = 32; bn = 1;
    int bt = wgs(32, 1);  // (32, 1) always fits
    for (int i = 0; i < 4; ++i) {
      const int* c = cand[i];
      if (mostly_padding(c[1])) continue;
      if (wgs(c[0], c[1]) > bt) { bw = c[0]; bn = c[1]; bt = wgs(c[0], c[1]); }
    }
    // at most one feature block per split on the per-slot kernel (one barrier per
    // slot: a shorter chain pays; 256 x 64 -> 64 fp32: 4 splits 9.0 us, 2 splits
    // 12.8 us), two on the block kernel
    const bool per_slot = block_waves(!f32, L->basis, bw, bn, KP) == 0;
    s = std::max(1, std::min((512 + bt - 1) / bt, std::max(1, per_slot ? L->nfb : L->nfb / 2)));
  }
  if (L->forced_wm && L->forced_nb) { bw = L->forced_wm; bn = L->forced_nb; }
  if (L->forced_splits) s = L->forced_splits;
  *wm = bw;
  *nb = bn;
  *splits = s;
}

// Wave groups per workgroup (KS) of the 4-wave block kernel for a forward of
// batch B on tile (wm, nb) x splits.  A layer that leaves at most one such
// workgroup per CU gets 4 groups on (32,1) or 2 on (32,4), when each group
// still has at least 4 feature blocks: one workgroup per CU then holds 4·KS
// waves instead of 4, each with a KS times shorter chain of blocks.  A forced
// tile keeps one group unless the groups are forced too; a forced count that
// the tile is not instantiated with falls back to 1.
static int choose_wave_groups(const kans_layer* L, int B, int wm, int nb, int splits) {
  if (block_waves(L->dtype != DT_F32, L->basis, wm, nb, L->K + L->has_base) != 4) return 1;
  if (L->forced_ks) return block_wave_groups_ok(wm, nb, L->forced_ks) ? L->forced_ks : 1;
  if (L->forced_wm) return 1;
  const long wgs = (long)((B + 4 * wm - 1) / (4 * wm)) * (((L->D_out + 31) / 32 + nb - 1) / nb) * splits;
  const int fbps = (L->nfb + splits - 1) / splits;
  if (wgs > 256) return 1;
  if (block_wave_groups_ok(wm, nb, 4) && fbps >= 16) return 4;
  if (block_wave_groups_ok(wm, nb, 2) && fbps >= 8) return 2;
  return 1;
}

// Reserve the split workspace a forward of batch B needs (no launch).
static int layer_reserve_locked(kans_layer* L, int B) {
  int wm, nb, splits;
  choose_tiling(L, B, &wm, &nb, &splits);
  if (splits > 1) {
    void* old = L->part.p;
    int rc = L->part.reserve((size_t)splits * B * L->D_out * sizeof(float));
    if (rc) return rc;
    if (old != L->part.p) ++L->gen;
  }
  return 0;
}

// Enqueue one fused forward; allocates nothing when layer_reserve_locked(L, B)
// ran before (the chain relies on this while capturing a graph).
// cfg_B > 0: use the tile configuration a forward of cfg_B rows would use (the
// chunked host forward launches row chunks of a batch with the whole batch's
// configuration, so every row gets the same result as in one launch).
static int layer_launch_locked(kans_layer* L, const void* X, long ldx, void* Y, long ldy, int B, hipStream_t st,
                               int x_dtype = -1, int y_dtype = -1, int cfg_B = 0) {
  if (x_dtype < 0) x_dtype = L->dtype;
  if (y_dtype < 0) y_dtype = L->dtype;
  if ((x_dtype != L->dtype && x_dtype != DT_F32) || (y_dtype != L->dtype && y_dtype != DT_F32))
    return kans_fail(KANS_ERR_ARG, "input/output dtype must be the layer dtype or fp32");
  if (!L->have_weights) return kans_fail(KANS_ERR_STATE, "layer has no weights loaded");
  if (L->basis == BASIS_RBF && !L->bp.have_centers) return kans_fail(KANS_ERR_STATE, "RBF centres not set");
  if (L->basis == BASIS_BSPLINE && L->bp.grid_size <= 0) return kans_fail(KANS_ERR_STATE, "B-spline grid not set");
  if (B <= 0) return 0;
  if (ldx < L->D_in8 || (ldx % 8) != 0)
    return kans_fail(KANS_ERR_ARG, "ldx=%ld must be >= %d and a multiple of 8", ldx, L->D_in8);
  if (x_dtype == DT_F32 && L->dtype != DT_F32 && ((uintptr_t)X & 31) != 0)
    return kans_fail(KANS_ERR_ARG, "fp32 X must be 32-byte aligned");
  if (ldy < L->D_out) return kans_fail(KANS_ERR_ARG, "ldy=%ld < D_out=%d", ldy, L->D_out);
  if (((uintptr_t)X & 15) != 0) return kans_fail(KANS_ERR_ARG, "X must be 16-byte aligned");
  DenseLaunch D{};
  D.dtype = L->dtype;
  D.x_dtype = x_dtype;
  D.y_dtype = y_dtype;
  D.basis = L->basis;
  D.has_base = L->has_base;
  D.X = X;
  D.ldx = ldx;
  D.Wt = L->Wt.p;
  D.nob_pad = L->nob_pad;
  D.bias = L->has_bias ? L->bias_d.p : nullptr;
  D.Y = Y;
  D.ldy = ldy;
  D.B = B;
  D.D_in = L->D_in;
  D.D_out = L->D_out;
  D.nfb = L->nfb;
  D.bp = L->bp;
  if (cfg_B <= 0) cfg_B = B;
  choose_tiling(L, cfg_B, &D.wm, &D.nb, &D.splits);
  D.ks = choose_wave_groups(L, cfg_B, D.wm, D.nb, D.splits);
  D.pair = L->block_pairs;
  if (D.splits > 1) {
    if (L->part.cap < (size_t)D.splits * B * L->D_out * sizeof(float))
      return kans_fail(KANS_ERR_STATE, "split workspace not reserved");
    D.part = (float*)L->part.p;
  }
  HIP_TRY(launch_dense(D, st));
  return 0;
}

static int layer_forward_locked(kans_layer* L, const void* X, long ldx, void* Y, long ldy, int B, hipStream_t st) {
  int rc = layer_reserve_locked(L, B);
  if (rc) return rc;
  return layer_launch_locked(L, X, ldx, Y, ldy, B, st);
}

// Large synchronous host forwards as a pipeline of row chunks: chunk c's input
// copy (g_copy_in), then its kernels (g_stream or g_compute2, alternating,
// after an event), then its output copy (g_copy_out, after an event), so that
// the PCIe transfers in both directions and the kernels of different chunks
// overlap; the host copies of chunk c + 1 run while the device works on
// chunk c.  Every chunk is launched with the tile configuration of the whole
// batch, which leaves each row's result exactly what one launch gives; only
// configurations without a feature split are chunked (no workspace is shared
// by chunk kernels that may run at the same time).  Chunks are whole 256-row
// tiles.  Measured on one MI355X, FastKAN fp16 16384 x 1024 -> 1024 from and
// into host arrays: 2.06 -> 1.54 ms per call (the C entry point, output array
// reused), 2.87 -> 1.92 ms through FastKAN.__call__ (a fresh output array).
constexpr size_t kChunkedBytes = size_t(16) << 20;  // x + y bytes from which a host forward is chunked
constexpr int kHostChunks = 4;
static std::vector<hipEvent_t> g_chunk_events;  // grow-only (library lock)

static int layer_forward_host_chunked(kans_layer* L, const void* X, void* Y, int B, int x_dtype) {
  const size_t es = dtype_size(L->dtype), xes = dtype_size(x_dtype);
  const long ldx = L->D_in8;
  const size_t row_in = (size_t)L->D_in * xes, pitch_in = (size_t)ldx * xes, row_out = (size_t)L->D_out * es;
  const int crow = (((B + kHostChunks - 1) / kHostChunks) + 255) / 256 * 256;
  const int n = (B + crow - 1) / crow;
  int rc;
  while ((int)g_chunk_events.size() < 2 * n + 1) {
    hipEvent_t e;
    HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    g_chunk_events.push_back(e);
  }
  // the side streams start after everything already on g_stream (a weight upload and its re-tiling
  // kernel, say); the call returns only after every chunk's output copy, so nothing outlives it
  hipEvent_t e0 = g_chunk_events[2 * n];
  HIP_TRY(hipEventRecord(e0, g_stream));
  HIP_TRY(hipStreamWaitEvent(g_copy_in, e0, 0));
  HIP_TRY(hipStreamWaitEvent(g_compute2, e0, 0));
  HIP_TRY(hipStreamWaitEvent(g_copy_out, e0, 0));
  char* xd = (char*)L->x_d.p;
  char* yd = (char*)L->y_d.p;
  char* pin_in = (char*)g_pin_in.p;
  char* pin_out = (char*)g_pin_out.p;
  StagedOut out;
  auto fail = [&](int code) {
    (void)hipStreamSynchronize(g_copy_in);
    (void)hipStreamSynchronize(g_stream);
    (void)hipStreamSynchronize(g_compute2);
    (void)hipStreamSynchronize(g_copy_out);
    return code;
  };
  for (int c = 0; c < n; ++c) {
    const long r0 = (long)c * crow;
    const int rows = (int)std::min<long>(crow, B - r0);
    hipEvent_t e_in = g_chunk_events[2 * c], e_k = g_chunk_events[2 * c + 1];
    hipStream_t cs = (c & 1) ? g_compute2 : g_stream;
    if ((rc = stage_in(xd + r0 * pitch_in, (const char*)X + r0 * row_in, row_in, pitch_in, rows,
                       pin_in + r0 * pitch_in, g_copy_in)))
      return fail(rc);
    if (hipEventRecord(e_in, g_copy_in) != hipSuccess || hipStreamWaitEvent(cs, e_in, 0) != hipSuccess)
      return fail(kans_fail(KANS_ERR_HIP, "chunked host forward: input event"));
    if ((rc = layer_launch_locked(L, xd + r0 * pitch_in, ldx, yd + r0 * row_out, L->D_out, rows, cs, x_dtype,
                                  L->dtype, B)))
      return fail(rc);
    if (hipEventRecord(e_k, cs) != hipSuccess || hipStreamWaitEvent(g_copy_out, e_k, 0) != hipSuccess)
      return fail(kans_fail(KANS_ERR_HIP, "chunked host forward: kernel event"));
    if ((rc = stage_out_enqueue(out, (char*)Y + r0 * row_out, yd + r0 * row_out, (size_t)rows * row_out,
                                pin_out + r0 * row_out, g_copy_out)))
      return fail(rc);
  }
  if ((rc = stage_out_drain(out))) return fail(rc);
  return 0;
}

// Host-memory forward: X [B][D_in] (layer dtype, or fp32 for a 16-bit layer)
// and Y [B][D_out] (layer dtype), contiguous; pinned staging.
static int layer_forward_host_locked(kans_layer* L, const void* X, void* Y, int B, int x_dtype = -1) {
  if (B <= 0) return 0;
  if (x_dtype < 0) x_dtype = L->dtype;
  const size_t es = dtype_size(L->dtype);
  const size_t xes = dtype_size(x_dtype);
  const long ldx = L->D_in8;
  const size_t xbytes = (size_t)B * ldx * xes;
  const size_t ybytes = (size_t)B * L->D_out * es;
  int rc;
  if ((rc = L->x_d.reserve(xbytes))) return rc;
  if ((rc = L->y_d.reserve(ybytes))) return rc;
  if ((rc = layer_reserve_locked(L, B))) return rc;
  // rows padded with zeros to a multiple of 8 features
  const size_t row_in = (size_t)L->D_in * xes, pitch_in = (size_t)ldx * xes;
  if (g_async) {  // per-call pinned buffers; the result lands in Y at metal_kan_sync
    void* pin_in;
    void* pin_out;
    HIP_TRY(hipHostMalloc(&pin_in, xbytes, hipHostMallocDefault));
    if (hipHostMalloc(&pin_out, ybytes, hipHostMallocDefault) != hipSuccess) {
      (void)hipHostFree(pin_in);
      return kans_fail(KANS_ERR_HIP, "hipHostMalloc of %zu bytes failed", ybytes);
    }
    // both buffers are freed at the next sync; Y is registered only once every step is enqueued
    g_pending.push_back({pin_in, nullptr, 0});
    g_pending.push_back({pin_out, nullptr, 0});
    const size_t out_idx = g_pending.size() - 1;
    if ((rc = stage_in(L->x_d.p, X, row_in, pitch_in, B, pin_in, g_stream))) return rc;
    if ((rc = layer_launch_locked(L, L->x_d.p, ldx, L->y_d.p, L->D_out, B, g_stream, x_dtype, L->dtype)))
      return rc;
    HIP_TRY(hipMemcpyAsync(pin_out, L->y_d.p, ybytes, hipMemcpyDeviceToHost, g_stream));
    g_pending[out_idx].dst = Y;
    g_pending[out_idx].bytes = ybytes;
    return 0;
  }
  if ((rc = pinned_reserve(g_pin_in, xbytes))) return rc;
  if ((rc = pinned_reserve(g_pin_out, ybytes))) return rc;
  if (xbytes + ybytes >= kChunkedBytes && B >= 2 * 256) {
    int wm, nb, splits;
    choose_tiling(L, B, &wm, &nb, &splits);
    if (splits == 1) return layer_forward_host_chunked(L, X, Y, B, x_dtype);
  }
  if ((rc = stage_in(L->x_d.p, X, row_in, pitch_in, B, g_pin_in.p, g_stream))) return rc;
  if ((rc = layer_launch_locked(L, L->x_d.p, ldx, L->y_d.p, L->D_out, B, g_stream, x_dtype, L->dtype))) {
    (void)hipStreamSynchronize(g_stream);  // the input DMAs read g_pin_in; finish them before it is reused
    return rc;
  }
  return stage_out(Y, L->y_d.p, ybytes, g_pin_out.p, g_stream);
}

static int sync_locked() {
  if (!g_ready) return 0;
  HIP_TRY(hipStreamSynchronize(g_stream));
  for (auto& p : g_pending) {
    if (p.dst) memcpy(p.dst, p.pinned, p.bytes);
    (void)hipHostFree(p.pinned);
  }
  g_pending.clear();
  return 0;
}

extern "C" {

int kans_layer_forward(kans_layer* L, const void* X, long ldx, void* Y, long ldy, int B, void* stream) {
  if (!L || !X || !Y) return kans_fail(KANS_ERR_ARG, "null argument");
  std::lock_guard<std::mutex> lk(g_mu);
  return layer_forward_locked(L, X, ldx, Y, ldy, B, stream ? (hipStream_t)stream : g_stream);
}

int kans_layer_forward_ex(kans_layer* L, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy, int B,
                          void* stream) {
  if (!L || !X || !Y) return kans_fail(KANS_ERR_ARG, "null argument");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = layer_reserve_locked(L, B);
  if (rc) return rc;
  return layer_launch_locked(L, X, ldx, Y, ldy, B, stream ? (hipStream_t)stream : g_stream, x_dtype, y_dtype);
}

int kans_layer_forward_host(kans_layer* L, const void* X, void* Y, int B) {
  if (!L || (B > 0 && (!X || !Y))) return kans_fail(KANS_ERR_ARG, "null argument");
  if (B < 0) return kans_fail(KANS_ERR_ARG, "B=%d < 0", B);
  std::lock_guard<std::mutex> lk(g_mu);
  return layer_forward_host_locked(L, X, Y, B);
}

int kans_layer_forward_host_ex(kans_layer* L, const void* X, int x_dtype, void* Y, int B) {
  if (!L || (B > 0 && (!X || !Y))) return kans_fail(KANS_ERR_ARG, "null argument");
  if (B < 0) return kans_fail(KANS_ERR_ARG, "B=%d < 0", B);
  if (x_dtype != L->dtype && x_dtype != DT_F32)
    return kans_fail(KANS_ERR_ARG, "x_dtype must be the layer dtype or fp32");
  std::lock_guard<std::mutex> lk(g_mu);
  return layer_forward_host_locked(L, X, Y, B, x_dtype);
}

int kans_layer_describe(const kans_layer* L, int B, int* wm, int* nb, int* splits) {
  if (!L || !wm || !nb || !splits) return kans_fail(KANS_ERR_ARG, "null argument");
  choose_tiling(L, B, wm, nb, splits);
  return 0;
}

// Name of the fused kernel a forward of batch B runs.  io = false: the layer dtype and basis variant
// ("kans::kan_fused_block<_Float16, BASIS_RBF_REC, 32, 8, 8 waves>"); io = true: the template's element
// types of X and Y as well, in template order ("kans::kan_fused_block<_Float16, _Float16, _Float16,
// BASIS_RBF_REC, 32, 8, 8 waves>"), as launch_dense routes x_dtype / y_dtype.
static int layer_kernel_name(const kans_layer* L, int B, bool io, int x_dtype, int y_dtype, char* name, int len) {
  int wm, nb, splits;
  choose_tiling(L, B, &wm, &nb, &splits);
  static const char* dt[] = {"float", "_Float16", "__bf16"};
  static const char* bs[] = {"BASIS_CHEBY", "BASIS_RBF", "BASIS_BSPLINE"};
  const int waves = block_waves(L->dtype != DT_F32, L->basis, wm, nb, L->K + L->has_base);
  const int ks = choose_wave_groups(L, B, wm, nb, splits);
  char groups[32] = "";
  if (ks > 1) snprintf(groups, sizeof groups, " x %d groups", ks);
  const bool pairs = waves == 8 && L->basis == BASIS_CHEBY && L->block_pairs && 2 * (L->K + L->has_base) <= 10;
  char types[64];
  if (io)
    snprintf(types, sizeof types, "%s, %s, %s", dt[L->dtype], dt[x_dtype == DT_F32 ? DT_F32 : L->dtype],
             dt[y_dtype == DT_F32 ? DT_F32 : L->dtype]);
  else
    snprintf(types, sizeof types, "%s", dt[L->dtype]);
  int n;
  if (waves)
    n = snprintf(name, len, "kans::kan_fused_block<%s, %s, %d, %d, %d waves%s>", types,
                 L->basis == BASIS_RBF       ? (L->bp.rbf_rec ? "BASIS_RBF_REC" : "BASIS_RBF_TABLE")
                 : L->basis == BASIS_BSPLINE && waves == 8 && L->bp.grid_size == kBsplineTabG
                     ? (L->has_base ? "BASIS_BSPLINE_TAB" : "BASIS_BSPLINE_TAB0")
                     : bs[L->basis],
                 wm, nb, waves, groups);
  else
    n = snprintf(name, len, "kans::kan_fused_dense<%s, %s, %d, %d>", types, bs[L->basis], wm, nb);
  if (n >= 0 && splits > 1)
    n += snprintf(name + std::min(n, len - 1), len - std::min(n, len - 1), " x %d feature splits", splits);
  if (n >= 0 && pairs) snprintf(name + std::min(n, len - 1), len - std::min(n, len - 1), ", 2 feature blocks per stage");
  return 0;
}

int kans_layer_kernel(const kans_layer* L, int B, char* name, int len) {
  if (!L || !name || len <= 0) return kans_fail(KANS_ERR_ARG, "null argument");
  return layer_kernel_name(L, B, false, L->dtype, L->dtype, name, len);
}

int kans_layer_kernel_ex(const kans_layer* L, int B, int x_dtype, int y_dtype, char* name, int len) {
  if (!L || !name || len <= 0) return kans_fail(KANS_ERR_ARG, "null argument");
  if ((x_dtype != L->dtype && x_dtype != DT_F32) || (y_dtype != L->dtype && y_dtype != DT_F32))
    return kans_fail(KANS_ERR_ARG, "input/output dtype must be the layer dtype or fp32");
  return layer_kernel_name(L, B, true, x_dtype, y_dtype, name, len);
}

// ---------------------------------------------------------------------------
// Device memory / stream / timing helpers (tests, benchmarks, integrations).
// ---------------------------------------------------------------------------
int kans_init(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  return ensure_init();
}

void* kans_stream(void) { return (void*)g_stream; }

int kans_dev_malloc(void** p, size_t bytes) {
  if (!p) return kans_fail(KANS_ERR_ARG, "null argument");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = ensure_init();
  if (rc) return rc;
  HIP_TRY(hipMalloc(p, bytes ? bytes : 16));
  return 0;
}

int kans_dev_free(void* p) {
  if (!p) return 0;
  HIP_TRY(hipFree(p));
  return 0;
}

int kans_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  if (!dst || !src) return kans_fail(KANS_ERR_ARG, "null argument");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = ensure_init();
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
  HIP_TRY(hipStreamSynchronize(g_stream));
  return 0;
}

int kans_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  if (!dst || !src) return kans_fail(KANS_ERR_ARG, "null argument");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = ensure_init();
  if (rc) return rc;
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
  HIP_TRY(hipStreamSynchronize(g_stream));
  return 0;
}

int kans_synchronize(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ready) return 0;
  HIP_TRY(hipStreamSynchronize(g_stream));
  return 0;
}

// Time `iters` back-to-back device-resident forwards with HIP events recorded on
// the stream the kernels run on; returns the mean per forward in *ms.
int kans_layer_time_forward(kans_layer* L, const void* X, long ldx, void* Y, long ldy, int B, int warmup,
                            int iters, float* ms) {
  if (!L || !X || !Y || !ms || iters <= 0) return kans_fail(KANS_ERR_ARG, "bad argument");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc;
  for (int i = 0; i < warmup; ++i)
    if ((rc = layer_forward_locked(L, X, ldx, Y, ldy, B, g_stream))) return rc;
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0));
  HIP_TRY(hipEventCreate(&e1));
  HIP_TRY(hipEventRecord(e0, g_stream));
  for (int i = 0; i < iters; ++i)
    if ((rc = layer_forward_locked(L, X, ldx, Y, ldy, B, g_stream))) return rc;
  HIP_TRY(hipEventRecord(e1, g_stream));
  HIP_TRY(hipEventSynchronize(e1));
  float t = 0;
  HIP_TRY(hipEventElapsedTime(&t, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *ms = t / iters;
  return 0;
}

// Clock-settled timing of one window: forwards run back to back for at least
// settle_ms of wall time (synchronised every 16 launches, so it is GPU time),
// then `iters` forwards are bracketed by stream synchronisation (wall clock)
// and, inside that bracket, by HIP events on the launch stream.  Both means
// come from the same launches, so *kernel_ms <= *wall_ms.
int kans_layer_time_window(kans_layer* L, const void* X, long ldx, void* Y, long ldy, int B, float settle_ms,
                           int iters, float* kernel_ms, float* wall_ms) {
  if (!L || !X || !Y || !kernel_ms || !wall_ms || iters <= 0 || !(settle_ms >= 0.0f))
    return kans_fail(KANS_ERR_ARG, "bad argument");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc;
  const auto s0 = std::chrono::steady_clock::now();
  do {
    for (int i = 0; i < 16; ++i)
      if ((rc = layer_forward_locked(L, X, ldx, Y, ldy, B, g_stream))) return rc;
    HIP_TRY(hipStreamSynchronize(g_stream));
  } while (std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - s0).count() < settle_ms);
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0));
  HIP_TRY(hipEventCreate(&e1));
  HIP_TRY(hipStreamSynchronize(g_stream));
  const auto t0 = std::chrono::steady_clock::now();
  HIP_TRY(hipEventRecord(e0, g_stream));
  for (int i = 0; i < iters; ++i)
    if ((rc = layer_forward_locked(L, X, ldx, Y, ldy, B, g_stream))) return rc;
  HIP_TRY(hipEventRecord(e1, g_stream));
  HIP_TRY(hipStreamSynchronize(g_stream));
  const auto t1 = std::chrono::steady_clock::now();
  float t = 0;
  HIP_TRY(hipEventElapsedTime(&t, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *kernel_ms = t / iters;
  *wall_ms = (float)(std::chrono::duration<double, std::milli>(t1 - t0).count() / iters);
  return 0;
}

// ---------------------------------------------------------------------------
// Reference-named entry points (metal_kans/device.py:64-474 argtypes).
// ---------------------------------------------------------------------------
int metal_kan_init(const char* /*shader_path: unused, kernels are compiled ahead of time*/) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = ensure_init();
  return rc ? -1 : 0;  // reference: -1 = no device (metal_kan_bridge.mm:293)
}

int metal_kan_set_async(int enabled) {
  g_async = enabled ? 1 : 0;
  return 0;
}

int metal_kan_sync(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  return sync_locked();
}

}  // extern "C"

// A layer per (shape, params) signature serves the reference-named calls; the
// caller's host weights are uploaded on every call (the reference reads them
// in place through zero-copy buffers, so in-place edits must be honoured).
typedef std::tuple<int, int, int, int, int, int, int, std::vector<float>> SigKey;
static std::map<SigKey, std::unique_ptr<kans_layer>> g_sig_layers;

static int sig_layer(int basis, int dtype, int D_in, int D_out, int K, int has_base, int has_bias,
                     const std::vector<float>& params, kans_layer** out) {
  if (basis == BASIS_RBF && !rbf_inv_den_ok(params[K]))
    return kans_fail(KANS_ERR_ARG, "RBF inv_denominator must be finite and >= 0");
  SigKey key(basis, dtype, D_in, D_out, K, has_base, has_bias, params);
  auto it = g_sig_layers.find(key);
  if (it != g_sig_layers.end()) {
    *out = it->second.get();
    return 0;
  }
  int rc = ensure_init();
  if (rc) return rc;
  auto L = std::make_unique<kans_layer>();
  L->basis = basis;
  L->dtype = dtype;
  L->D_in = D_in;
  L->D_out = D_out;
  L->K = K;
  L->has_base = has_base;
  L->has_bias = has_bias;
  L->D_in8 = round_up(D_in, 8);
  L->nfb = (D_in + 15) / 16;
  L->nob_pad = round_up((D_out + 31) / 32, kObPad);
  L->bp.K = K;
  if (basis == BASIS_RBF) {
    for (int k = 0; k < K; ++k) L->bp.centers[k] = params[k];
    L->bp.have_centers = 1;
    L->bp.neg_l = -params[K] * kLog2e;
    set_rbf_table(L->bp);
  } else if (basis == BASIS_BSPLINE) {
    L->bp.grid_size = K - 3;
    L->bp.grid_min = params[0];
    L->bp.inv_h = params[1];
  }
  if (g_sig_layers.size() > 64) g_sig_layers.clear();
  *out = L.get();
  g_sig_layers.emplace(key, std::move(L));
  return 0;
}

static int ref_forward(int basis, int dtype, const void* X, const void* W, const void* Wb, const void* bias, void* Y,
                       int B, int D_in, int D_out, int K, int has_base, int has_bias,
                       const std::vector<float>& params) {
  if (!X || !W || !Y) return kans_fail(KANS_ERR_ARG, "null X, W or Y");
  if (B < 0) return kans_fail(KANS_ERR_ARG, "B=%d < 0", B);
  int rc = validate_dims(basis, dtype, D_in, D_out, K, has_base, has_bias);
  if (rc) return rc;
  if (has_base && !Wb) return kans_fail(KANS_ERR_ARG, "has_base=1 but W_base is null");
  if (has_bias && !bias) return kans_fail(KANS_ERR_ARG, "has_bias=1 but bias is null");
  std::lock_guard<std::mutex> lk(g_mu);
  kans_layer* L;
  if ((rc = sig_layer(basis, dtype, D_in, D_out, K, has_base, has_bias, params, &L))) return rc;
  if ((rc = layer_upload_locked(L, W, Wb, bias, false, dtype))) return rc;
  return layer_forward_host_locked(L, X, Y, B);
}

// fp32 Chebyshev forward without a base branch of host X on device-resident fp32 weights W_dev
// [D_out][D_in*K] and bias_dev (device; null when !has_bias), through the same per-signature layer as
// the reference-named calls.  Lock held.  For weights produced on the device
// (metal_kan_forward_ternary_cheby): they are re-tiled from device memory, with no host copy.
int kans_ref_cheby_forward_devw_locked(const float* X, const float* W_dev, const float* bias_dev, float* Y, int B,
                                       int D_in, int D_out, int K, int has_bias) {
  if (!X || !W_dev || !Y || (has_bias && !bias_dev)) return kans_fail(KANS_ERR_ARG, "null argument");
  if (B < 0) return kans_fail(KANS_ERR_ARG, "B=%d < 0", B);
  int rc = validate_dims(BASIS_CHEBY, DT_F32, D_in, D_out, K, 0, has_bias);
  if (rc) return rc;
  kans_layer* L;
  if ((rc = sig_layer(BASIS_CHEBY, DT_F32, D_in, D_out, K, 0, has_bias, {}, &L))) return rc;
  if ((rc = layer_upload_locked(L, W_dev, nullptr, bias_dev, true, DT_F32))) return rc;
  return layer_forward_host_locked(L, X, Y, B);
}

static void half_to_floats(const uint16_t* h, float* f, int n) {
  for (int i = 0; i < n; ++i) {
    _Float16 v;
    memcpy(&v, &h[i], 2);
    f[i] = (float)v;
  }
}

extern "C" {

int metal_kan_cheby_forward(const float* X, const float* W, const float* Wb, const float* bias, float* Y, int B,
                            int D_in, int D_out, int K, int has_base, int has_bias) {
  return ref_forward(BASIS_CHEBY, DT_F32, X, W, Wb, bias, Y, B, D_in, D_out, K, has_base, has_bias, {});
}
int metal_kan_cheby_forward_fp16(const uint16_t* X, const uint16_t* W, const uint16_t* Wb, const uint16_t* bias,
                                 uint16_t* Y, int B, int D_in, int D_out, int K, int has_base, int has_bias) {
  return ref_forward(BASIS_CHEBY, DT_F16, X, W, Wb, bias, Y, B, D_in, D_out, K, has_base, has_bias, {});
}
int metal_kan_cheby_forward_bf16(const uint16_t* X, const uint16_t* W, const uint16_t* Wb, const uint16_t* bias,
                                 uint16_t* Y, int B, int D_in, int D_out, int K, int has_base, int has_bias) {
  return ref_forward(BASIS_CHEBY, DT_BF16, X, W, Wb, bias, Y, B, D_in, D_out, K, has_base, has_bias, {});
}

int metal_kan_fastkan_forward(const float* X, const float* W, const float* Wb, const float* grid, const float* bias,
                              float* Y, int B, int D_in, int D_out, int K, float inv_den, int has_base,
                              int has_bias) {
  if (!grid || K <= 0 || K > kMaxK) return kans_fail(KANS_ERR_ARG, "null grid or bad K");
  std::vector<float> p(grid, grid + K);
  p.push_back(inv_den);
  return ref_forward(BASIS_RBF, DT_F32, X, W, Wb, bias, Y, B, D_in, D_out, K, has_base, has_bias, p);
}
int metal_kan_fastkan_forward_fp16(const uint16_t* X, const uint16_t* W, const uint16_t* Wb, const uint16_t* grid,
                                   const uint16_t* bias, uint16_t* Y, int B, int D_in, int D_out, int K,
                                   float inv_den, int has_base, int has_bias) {
  if (!grid || K <= 0 || K > kMaxK) return kans_fail(KANS_ERR_ARG, "null grid or bad K");
  std::vector<float> p(K);
  half_to_floats(grid, p.data(), K);
  p.push_back(inv_den);
  return ref_forward(BASIS_RBF, DT_F16, X, W, Wb, bias, Y, B, D_in, D_out, K, has_base, has_bias, p);
}
int metal_kan_fastkan_forward_bf16(const uint16_t* X, const uint16_t* W, const uint16_t* Wb, const float* grid,
                                   const uint16_t* bias, uint16_t* Y, int B, int D_in, int D_out, int K,
                                   float inv_den, int has_base, int has_bias) {
  if (!grid || K <= 0 || K > kMaxK) return kans_fail(KANS_ERR_ARG, "null grid or bad K");
  std::vector<float> p(grid, grid + K);
  p.push_back(inv_den);
  return ref_forward(BASIS_RBF, DT_BF16, X, W, Wb, bias, Y, B, D_in, D_out, K, has_base, has_bias, p);
}

static int bspline_common(int dtype, const void* X, const void* W, const void* Wb, const float* grid,
                          const void* bias, void* Y, int B, int D_in, int D_out, int G, int has_base,
                          int has_bias) {
  if (!grid) return kans_fail(KANS_ERR_ARG, "null grid params");
  if (G <= 0 || G + 3 > kMaxK) return kans_fail(KANS_ERR_ARG, "grid_size=%d out of range", G);
  std::vector<float> p{grid[0], grid[1]};
  return ref_forward(BASIS_BSPLINE, dtype, X, W, Wb, bias, Y, B, D_in, D_out, G + 3, has_base, has_bias, p);
}

// grid = [grid_min, inv_h] (fp32, read on the host as metal_kan_bridge.mm:1138-1139 does);
// spline_order is accepted and ignored, as in the reference (always cubic).
int metal_kan_bspline_forward(const float* X, const float* W, const float* Wb, const float* grid, const float* bias,
                              float* Y, int B, int D_in, int D_out, int G, int /*spline_order*/, int has_base,
                              int has_bias) {
  return bspline_common(DT_F32, X, W, Wb, grid, bias, Y, B, D_in, D_out, G, has_base, has_bias);
}
int metal_kan_bspline_forward_fp16(const uint16_t* X, const uint16_t* W, const uint16_t* Wb, const float* grid,
                                   const uint16_t* bias, uint16_t* Y, int B, int D_in, int D_out, int G,
                                   int /*spline_order*/, int has_base, int has_bias) {
  return bspline_common(DT_F16, X, W, Wb, grid, bias, Y, B, D_in, D_out, G, has_base, has_bias);
}
int metal_kan_bspline_forward_bf16(const uint16_t* X, const uint16_t* W, const uint16_t* Wb, const float* grid,
                                   const uint16_t* bias, uint16_t* Y, int B, int D_in, int D_out, int G,
                                   int /*spline_order*/, int has_base, int has_bias) {
  return bspline_common(DT_BF16, X, W, Wb, grid, bias, Y, B, D_in, D_out, G, has_base, has_bias);
}

// Wall-clock per full host call, warmup then iters (metal_kan_bridge.mm:1250-1277).
double benchmark_metal_cheby(const float* X, const float* W, const float* Wb, const float* bias, float* Y, int B,
                             int D_in, int D_out, int K, int has_base, int has_bias, int warmup, int iters) {
  for (int i = 0; i < warmup; ++i)
    if (metal_kan_cheby_forward(X, W, Wb, bias, Y, B, D_in, D_out, K, has_base, has_bias)) return -1.0;
  auto t0 = std::chrono::steady_clock::now();
  for (int i = 0; i < iters; ++i)
    if (metal_kan_cheby_forward(X, W, Wb, bias, Y, B, D_in, D_out, K, has_base, has_bias)) return -1.0;
  auto t1 = std::chrono::steady_clock::now();
  return std::chrono::duration<double, std::milli>(t1 - t0).count() / (iters > 0 ? iters : 1);
}

double benchmark_metal_fastkan(const float* X, const float* W, const float* Wb, const float* grid, const float* bias,
                               float* Y, int B, int D_in, int D_out, int K, float inv_den, int has_base,
                               int has_bias, int warmup, int iters) {
  for (int i = 0; i < warmup; ++i)
    if (metal_kan_fastkan_forward(X, W, Wb, grid, bias, Y, B, D_in, D_out, K, inv_den, has_base, has_bias))
      return -1.0;
  auto t0 = std::chrono::steady_clock::now();
  for (int i = 0; i < iters; ++i)
    if (metal_kan_fastkan_forward(X, W, Wb, grid, bias, Y, B, D_in, D_out, K, inv_den, has_base, has_bias))
      return -1.0;
  auto t1 = std::chrono::steady_clock::now();
  return std::chrono::duration<double, std::milli>(t1 - t0).count() / (iters > 0 ? iters : 1);
}

double benchmark_metal_bspline(const float* X, const float* W, const float* Wb, const float* grid, const float* bias,
                               float* Y, int B, int D_in, int D_out, int G, int order, int has_base, int has_bias,
                               int warmup, int iters) {
  for (int i = 0; i < warmup; ++i)
    if (metal_kan_bspline_forward(X, W, Wb, grid, bias, Y, B, D_in, D_out, G, order, has_base, has_bias))
      return -1.0;
  auto t0 = std::chrono::steady_clock::now();
  for (int i = 0; i < iters; ++i)
    if (metal_kan_bspline_forward(X, W, Wb, grid, bias, Y, B, D_in, D_out, G, order, has_base, has_bias))
      return -1.0;
  auto t1 = std::chrono::steady_clock::now();
  return std::chrono::duration<double, std::milli>(t1 - t0).count() / (iters > 0 ? iters : 1);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Multi-layer chain (replaces metal_kan_chain_pipeline_cheby,
// metal_kan_bridge.mm:1168-1248, which is fp32 / K=4 only and allocates its
// ping-pong buffers per call).  Device-resident ping-pong activations; the
// host path (H2D, every layer, D2H) is captured once per batch size as a HIP
// graph and replayed.
// ---------------------------------------------------------------------------
struct kans_chain {
  std::vector<kans_layer*> layers;
  std::vector<std::unique_ptr<kans_layer>> owned;  // layers created by metal_kan_chain_pipeline_cheby
  int dtype = 0;
  int mid_dtype = 0;  // activations between layers: fp32 (also for 16-bit chains)
  long ld_in = 0, ld_mid = 0, ld_out = 0;
  int cap_B = 0;
  DevBuf x_d, ping, pong, y_d;
  Pinned pin_in, pin_out;
  int in_dtype = 0;  // element type of the chain input (chain dtype or fp32)
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int graph_B = -1;
  int graph_in = -1;
  unsigned graph_gen = 0;
  bool graph_copies = false;
  ~kans_chain() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (pin_in.p) (void)hipHostFree(pin_in.p);
    if (pin_out.p) (void)hipHostFree(pin_out.p);
  }
};

static unsigned chain_gen(const kans_chain* C) {
  unsigned g = 0;
  for (auto* L : C->layers) g = g * 31u + L->gen;
  return g;
}

static int chain_reserve(kans_chain* C, int B) {
  int rc;
  for (auto* L : C->layers)
    if (L->dtype != C->dtype)
      return kans_fail(KANS_ERR_STATE, "a chain layer's dtype changed since kans_chain_create");
  if (B > C->cap_B) {
    const size_t es = dtype_size(C->dtype);
    void* olds[4] = {C->x_d.p, C->ping.p, C->pong.p, C->y_d.p};
    if ((rc = C->x_d.reserve((size_t)B * C->ld_in * 4))) return rc;  // room for an fp32 input
    const size_t ms = dtype_size(C->mid_dtype);
    if ((rc = C->ping.reserve((size_t)B * C->ld_mid * ms))) return rc;
    if ((rc = C->pong.reserve((size_t)B * C->ld_mid * ms))) return rc;
    if ((rc = C->y_d.reserve((size_t)B * C->ld_out * es))) return rc;
    // padding columns must hold finite values; zero everything once, outside any graph
    HIP_TRY(hipMemsetAsync(C->x_d.p, 0, C->x_d.cap, g_stream));
    HIP_TRY(hipMemsetAsync(C->ping.p, 0, C->ping.cap, g_stream));
    HIP_TRY(hipMemsetAsync(C->pong.p, 0, C->pong.cap, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    if ((rc = pinned_reserve(C->pin_in, (size_t)B * C->ld_in * 4))) return rc;
    if ((rc = pinned_reserve(C->pin_out, (size_t)B * C->ld_out * es))) return rc;
    C->cap_B = B;
    void* news[4] = {C->x_d.p, C->ping.p, C->pong.p, C->y_d.p};
    for (int i = 0; i < 4; ++i)
      if (olds[i] != news[i]) C->graph_B = -1;
  }
  for (auto* L : C->layers)
    if ((rc = layer_reserve_locked(L, B))) return rc;
  return 0;
}

// Enqueue all layers: X (ldx) -> ... -> Y (ldy) through the ping-pong buffers.
static int chain_launch(kans_chain* C, const void* X, long ldx, void* Y, long ldy, int B, hipStream_t st) {
  const void* src = X;
  long lds = ldx;
  const size_t n = C->layers.size();
  for (size_t l = 0; l < n; ++l) {
    void* dst = (l + 1 == n) ? Y : ((l % 2 == 0) ? C->pong.p : C->ping.p);
    long ldd = (l + 1 == n) ? ldy : C->ld_mid;
    const int xdt = (l == 0) ? C->in_dtype : C->mid_dtype;
    const int ydt = (l + 1 == n) ? C->dtype : C->mid_dtype;
    int rc = layer_launch_locked(C->layers[l], src, lds, dst, ldd, B, st, xdt, ydt);
    if (rc) return rc;
    src = dst;
    lds = ldd;
  }
  return 0;
}

static int chain_capture(kans_chain* C, int B, bool copies) {
  if (C->exec) { (void)hipGraphExecDestroy(C->exec); C->exec = nullptr; }
  if (C->graph) { (void)hipGraphDestroy(C->graph); C->graph = nullptr; }
  const size_t es = dtype_size(C->dtype);
  const size_t ies = dtype_size(C->in_dtype);
  HIP_TRY(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal));
  int rc = 0;
  if (copies) {
    hipError_t e = hipMemcpyAsync(C->x_d.p, C->pin_in.p, (size_t)B * C->ld_in * ies, hipMemcpyHostToDevice, g_stream);
    if (e != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "capture H2D: %s", hipGetErrorString(e));
  }
  if (!rc) rc = chain_launch(C, C->x_d.p, C->ld_in, C->y_d.p, C->ld_out, B, g_stream);
  if (!rc && copies) {
    hipError_t e = hipMemcpyAsync(C->pin_out.p, C->y_d.p, (size_t)B * C->ld_out * es, hipMemcpyDeviceToHost,
                                  g_stream);
    if (e != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "capture D2H: %s", hipGetErrorString(e));
  }
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(g_stream, &g);
  if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
  if (e != hipSuccess) return kans_fail(KANS_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
  C->graph = g;
  HIP_TRY(hipGraphInstantiate(&C->exec, C->graph, nullptr, nullptr, 0));
  C->graph_B = B;
  C->graph_in = C->in_dtype;
  C->graph_gen = chain_gen(C);
  C->graph_copies = copies;
  return 0;
}

static int chain_graph_ready(kans_chain* C, int B, bool copies) {
  int rc = chain_reserve(C, B);
  if (rc) return rc;
  if (C->exec && C->graph_B == B && C->graph_in == C->in_dtype && C->graph_gen == chain_gen(C) &&
      C->graph_copies == copies)
    return 0;
  return chain_capture(C, B, copies);
}

extern "C" {

int kans_chain_create(kans_layer** layers, int n, kans_chain** out) {
  if (!layers || n <= 0 || !out) return kans_fail(KANS_ERR_ARG, "bad chain arguments");
  for (int i = 0; i < n; ++i)
    if (!layers[i]) return kans_fail(KANS_ERR_ARG, "null layer %d", i);
  for (int i = 0; i + 1 < n; ++i) {
    if (layers[i]->D_out != layers[i + 1]->D_in)
      return kans_fail(KANS_ERR_ARG, "layer %d D_out=%d != layer %d D_in=%d", i, layers[i]->D_out, i + 1,
                       layers[i + 1]->D_in);
    if (layers[i]->dtype != layers[i + 1]->dtype) return kans_fail(KANS_ERR_ARG, "mixed dtypes in chain");
  }
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = ensure_init();
  if (rc) return rc;
  auto* C = new kans_chain();
  C->layers.assign(layers, layers + n);
  C->dtype = layers[0]->dtype;
  C->in_dtype = C->dtype;
  C->mid_dtype = DT_F32;
  C->ld_in = layers[0]->D_in8;
  long mid = 8;
  for (int i = 0; i + 1 < n; ++i) mid = std::max<long>(mid, round_up(layers[i]->D_out, 8));
  C->ld_mid = mid;
  C->ld_out = layers[n - 1]->D_out;
  *out = C;
  return 0;
}

int kans_chain_destroy(kans_chain* C) {
  if (!C) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ready) (void)hipStreamSynchronize(g_stream);
  delete C;
  return 0;
}

// Host arrays [B][D_in0] (x_dtype: chain dtype, or fp32) -> [B][D_out_last]
// (chain dtype), one graph replay.
int kans_chain_forward_host_ex(kans_chain* C, const void* X, int x_dtype, void* Y, int B) {
  if (!C || (B > 0 && (!X || !Y)) || B < 0) return kans_fail(KANS_ERR_ARG, "bad argument");
  if (x_dtype != C->dtype && x_dtype != DT_F32) return kans_fail(KANS_ERR_ARG, "x_dtype must be the chain dtype or fp32");
  if (B == 0) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  C->in_dtype = x_dtype;
  // the kernels-only graph; the host arrays are staged around it (stage_in / stage_out)
  int rc = chain_graph_ready(C, B, false);
  if (rc) return rc;
  const size_t es = dtype_size(C->dtype);
  const size_t xes = dtype_size(x_dtype);
  const int D0 = C->layers[0]->D_in;
  const size_t in_bytes = (size_t)B * C->ld_in * xes, out_bytes = (size_t)B * C->ld_out * es;
  const size_t row_in = (size_t)D0 * xes, pitch_in = (size_t)C->ld_in * xes;
  if (g_async) {  // per-call pinned buffers; the result lands in Y at metal_kan_sync
    void* pin_in;
    void* pin_out;
    HIP_TRY(hipHostMalloc(&pin_in, in_bytes, hipHostMallocDefault));
    if (hipHostMalloc(&pin_out, out_bytes, hipHostMallocDefault) != hipSuccess) {
      (void)hipHostFree(pin_in);
      return kans_fail(KANS_ERR_HIP, "hipHostMalloc of %zu bytes failed", out_bytes);
    }
    // both buffers are freed at the next sync; Y is registered only once every step is enqueued
    g_pending.push_back({pin_in, nullptr, 0});
    g_pending.push_back({pin_out, nullptr, 0});
    const size_t out_idx = g_pending.size() - 1;
    if ((rc = stage_in(C->x_d.p, X, row_in, pitch_in, B, pin_in, g_stream))) return rc;
    HIP_TRY(hipGraphLaunch(C->exec, g_stream));
    HIP_TRY(hipMemcpyAsync(pin_out, C->y_d.p, out_bytes, hipMemcpyDeviceToHost, g_stream));
    g_pending[out_idx].dst = Y;
    g_pending[out_idx].bytes = out_bytes;
    return 0;
  }
  if ((rc = stage_in(C->x_d.p, X, row_in, pitch_in, B, C->pin_in.p, g_stream))) return rc;
  if (hipGraphLaunch(C->exec, g_stream) != hipSuccess) {
    (void)hipStreamSynchronize(g_stream);  // the input DMAs read pin_in; finish them before it is reused
    return kans_fail(KANS_ERR_HIP, "hipGraphLaunch failed");
  }
  return stage_out(Y, C->y_d.p, out_bytes, C->pin_out.p, g_stream);
}

int kans_chain_forward_host(kans_chain* C, const void* X, void* Y, int B) {
  return kans_chain_forward_host_ex(C, X, C ? C->dtype : 0, Y, B);
}

// Device arrays: X [B][ldx] (ldx >= round_up(D_in0, 8), multiple of 8), Y [B][ldy]; eager launches.
int kans_chain_forward(kans_chain* C, const void* X, long ldx, void* Y, long ldy, int B, void* stream) {
  if (!C || !X || !Y || B < 0) return kans_fail(KANS_ERR_ARG, "bad argument");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = chain_reserve(C, B);
  if (rc) return rc;
  C->in_dtype = C->dtype;
  return chain_launch(C, X, ldx, Y, ldy, B, stream ? (hipStream_t)stream : g_stream);
}

// Time `iters` replays of the chain graph; include_copies = 1 also replays the
// pinned H2D / D2H copies.  *ms = mean per replay (HIP events on the stream).
int kans_chain_time(kans_chain* C, int B, int warmup, int iters, int include_copies, float* ms) {
  if (!C || B <= 0 || iters <= 0 || !ms) return kans_fail(KANS_ERR_ARG, "bad argument");
  std::lock_guard<std::mutex> lk(g_mu);  // replays the graph of the last host call's input dtype
  int rc = chain_graph_ready(C, B, include_copies != 0);
  if (rc) return rc;
  for (int i = 0; i < warmup; ++i) HIP_TRY(hipGraphLaunch(C->exec, g_stream));
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0));
  HIP_TRY(hipEventCreate(&e1));
  HIP_TRY(hipEventRecord(e0, g_stream));
  for (int i = 0; i < iters; ++i) HIP_TRY(hipGraphLaunch(C->exec, g_stream));
  HIP_TRY(hipEventRecord(e1, g_stream));
  HIP_TRY(hipEventSynchronize(e1));
  float t = 0;
  HIP_TRY(hipEventElapsedTime(&t, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *ms = t / iters;
  return 0;
}

// Reference-named fp32 Chebyshev chain (device.py:116-122): host weights are
// read on every call (uploaded into the chain's own layers), the activations
// never leave the device between layers.  A null W_bases[l] / biases[l]
// disables that branch for layer l, as in the reference.  Generalises the
// reference (any K per layer, not only 4).
typedef std::vector<int> ChainKey;
static std::map<ChainKey, std::unique_ptr<kans_chain>> g_ref_chains;

int metal_kan_chain_pipeline_cheby(const float* X, float* Y, int B, int num_layers, const int* dims,
                                   const int* degrees, const float** W_chebys, const float** W_bases,
                                   const float** biases) {
  if (!X || !Y || B < 0 || num_layers <= 0 || !dims || !degrees || !W_chebys)
    return kans_fail(KANS_ERR_ARG, "chain: bad argument");
  ChainKey key;
  for (int l = 0; l < num_layers; ++l) {
    if (!W_chebys[l]) return kans_fail(KANS_ERR_ARG, "chain: null W_cheby[%d]", l);
    int rc = validate_dims(BASIS_CHEBY, DT_F32, dims[l], dims[l + 1], degrees[l], 0, 0);
    if (rc) return rc;
    key.insert(key.end(), {dims[l], dims[l + 1], degrees[l], (W_bases && W_bases[l]) ? 1 : 0,
                           (biases && biases[l]) ? 1 : 0});
  }
  if (B == 0) return 0;
  kans_chain* C = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_init();
    if (rc) return rc;
    auto it = g_ref_chains.find(key);
    if (it == g_ref_chains.end()) {
      auto ch = std::make_unique<kans_chain>();
      for (int l = 0; l < num_layers; ++l) {
        auto L = std::make_unique<kans_layer>();
        L->basis = BASIS_CHEBY;
        L->dtype = DT_F32;
        L->D_in = dims[l];
        L->D_out = dims[l + 1];
        L->K = degrees[l];
        L->has_base = key[5 * l + 3];
        L->has_bias = key[5 * l + 4];
        L->D_in8 = round_up(L->D_in, 8);
        L->nfb = (L->D_in + 15) / 16;
        L->nob_pad = round_up((L->D_out + 31) / 32, kObPad);
        L->bp.K = L->K;
        ch->layers.push_back(L.get());
        ch->owned.push_back(std::move(L));
      }
      ch->dtype = DT_F32;
      ch->in_dtype = DT_F32;
      ch->mid_dtype = DT_F32;
      ch->ld_in = ch->layers[0]->D_in8;
      long mid = 8;
      for (int l = 0; l + 1 < num_layers; ++l) mid = std::max<long>(mid, round_up(dims[l + 1], 8));
      ch->ld_mid = mid;
      ch->ld_out = dims[num_layers];
      if (g_ref_chains.size() > 16) g_ref_chains.clear();
      it = g_ref_chains.emplace(key, std::move(ch)).first;
    }
    C = it->second.get();
    for (int l = 0; l < num_layers; ++l) {
      kans_layer* L = C->layers[l];
      rc = layer_upload_locked(L, W_chebys[l], L->has_base ? W_bases[l] : nullptr, L->has_bias ? biases[l] : nullptr,
                               false, DT_F32);
      if (rc) return rc;
    }
  }
  return kans_chain_forward_host(C, X, Y, B);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Dense GatedKAN block (gated_kan.py:86-138): gate(x), up(x), SiLU(gate)*up
// with the +-20 clip, down(hidden), all on device activations in the layers'
// dtype (a 16-bit block stores its gate / up / hidden activations in 16 bits,
// as its layers' outputs are).  The host path is one captured HIP graph per
// batch size: the pinned H2D copy of x, four kernels (the layers' fused
// forwards and the SwiGLU pass) and the D2H copy of y; async mode replays the
// kernels only and defers the copy into the caller's array to
// metal_kan_sync(), as the chain does.  Replaces the reference's four blocking
// submissions with host round trips between them.
// ---------------------------------------------------------------------------
namespace {

// hidden = (g * sigmoid(clamp(g, -20, 20))) * u in fp32 (fused_kan.metal:2284-2296,
// the arithmetic of metal_kan_swiglu_forward), stored in T.
template <typename T>
__global__ void k_gated_swiglu(const T* __restrict__ g, const T* __restrict__ u, T* __restrict__ out, long ld,
                               int rows, int cols) {
  const long n = (long)rows * cols;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x) {
    const long r = i / cols, c = i - r * cols;
    const long k = r * ld + c;
    const float gv = to_f32(g[k]);
    const float cl = fminf(fmaxf(gv, -20.0f), 20.0f);
    const float sig = 1.0f / (1.0f + expf(-cl));
    out[k] = from_f32<T>((gv * sig) * to_f32(u[k]));
  }
}

hipError_t launch_gated_swiglu(int dtype, const void* g, const void* u, void* out, long ld, int rows, int cols,
                               hipStream_t st) {
  const long n = (long)rows * cols;
  const int blocks = (int)std::min<long>((n + 255) / 256, 8192);
  if (dtype == DT_F16)
    hipLaunchKernelGGL(k_gated_swiglu<_Float16>, dim3(blocks), dim3(256), 0, st, (const _Float16*)g,
                       (const _Float16*)u, (_Float16*)out, ld, rows, cols);
  else if (dtype == DT_BF16)
    hipLaunchKernelGGL(k_gated_swiglu<__bf16>, dim3(blocks), dim3(256), 0, st, (const __bf16*)g, (const __bf16*)u,
                       (__bf16*)out, ld, rows, cols);
  else
    hipLaunchKernelGGL(k_gated_swiglu<float>, dim3(blocks), dim3(256), 0, st, (const float*)g, (const float*)u,
                       (float*)out, ld, rows, cols);
  return hipGetLastError();
}

}  // namespace

struct kans_gated_dense {
  kans_layer *gate, *up, *down;
  int dtype, d, h;
  long ld_in, ld_h, ld_out;
  int cap_B = 0;
  DevBuf x_d, g_d, u_d, h_d, y_d;
  Pinned pin_in, pin_out;
  int in_dtype = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int graph_B = -1, graph_in = -1;
  unsigned graph_gen = 0;
  bool graph_copies = false;
  ~kans_gated_dense() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (pin_in.p) (void)hipHostFree(pin_in.p);
    if (pin_out.p) (void)hipHostFree(pin_out.p);
  }
};

static unsigned dgated_gen(const kans_gated_dense* D) {
  return (D->gate->gen * 31u + D->up->gen) * 31u + D->down->gen;
}

static int dgated_reserve(kans_gated_dense* D, int B) {
  int rc;
  for (const kans_layer* L : {D->gate, D->up, D->down})
    if (L->dtype != D->dtype)
      return kans_fail(KANS_ERR_STATE, "a block layer's dtype changed since kans_gated_dense_create");
  if (B > D->cap_B) {
    const size_t es = dtype_size(D->dtype);
    void* olds[5] = {D->x_d.p, D->g_d.p, D->u_d.p, D->h_d.p, D->y_d.p};
    if ((rc = D->x_d.reserve((size_t)B * D->ld_in * 4))) return rc;  // room for an fp32 input
    if ((rc = D->g_d.reserve((size_t)B * D->ld_h * es))) return rc;
    if ((rc = D->u_d.reserve((size_t)B * D->ld_h * es))) return rc;
    if ((rc = D->h_d.reserve((size_t)B * D->ld_h * es))) return rc;
    if ((rc = D->y_d.reserve((size_t)B * D->ld_out * es))) return rc;
    // padding columns read as inputs: zero them once, outside any graph
    HIP_TRY(hipMemsetAsync(D->x_d.p, 0, D->x_d.cap, g_stream));
    HIP_TRY(hipMemsetAsync(D->h_d.p, 0, D->h_d.cap, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    if ((rc = pinned_reserve(D->pin_in, (size_t)B * D->ld_in * 4))) return rc;
    if ((rc = pinned_reserve(D->pin_out, (size_t)B * D->ld_out * es))) return rc;
    D->cap_B = B;
    void* news[5] = {D->x_d.p, D->g_d.p, D->u_d.p, D->h_d.p, D->y_d.p};
    for (int i = 0; i < 5; ++i)
      if (olds[i] != news[i]) D->graph_B = -1;
  }
  for (kans_layer* L : {D->gate, D->up, D->down})
    if ((rc = layer_reserve_locked(L, B))) return rc;
  return 0;
}

// Enqueue gate, up, SwiGLU and down: X (x_dtype, ldx) -> Y (block dtype, ldy).
static int dgated_launch(kans_gated_dense* D, const void* X, int x_dtype, long ldx, void* Y, long ldy, int B,
                         hipStream_t st) {
  int rc;
  if ((rc = layer_launch_locked(D->gate, X, ldx, D->g_d.p, D->ld_h, B, st, x_dtype, D->dtype))) return rc;
  if ((rc = layer_launch_locked(D->up, X, ldx, D->u_d.p, D->ld_h, B, st, x_dtype, D->dtype))) return rc;
  HIP_TRY(launch_gated_swiglu(D->dtype, D->g_d.p, D->u_d.p, D->h_d.p, D->ld_h, B, D->h, st));
  return layer_launch_locked(D->down, D->h_d.p, D->ld_h, Y, ldy, B, st, D->dtype, D->dtype);
}

static int dgated_capture(kans_gated_dense* D, int B, bool copies) {
  if (D->exec) { (void)hipGraphExecDestroy(D->exec); D->exec = nullptr; }
  if (D->graph) { (void)hipGraphDestroy(D->graph); D->graph = nullptr; }
  const size_t es = dtype_size(D->dtype), ies = dtype_size(D->in_dtype);
  HIP_TRY(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal));
  int rc = 0;
  if (copies) {
    hipError_t e = hipMemcpyAsync(D->x_d.p, D->pin_in.p, (size_t)B * D->ld_in * ies, hipMemcpyHostToDevice, g_stream);
    if (e != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "capture H2D: %s", hipGetErrorString(e));
  }
  if (!rc) rc = dgated_launch(D, D->x_d.p, D->in_dtype, D->ld_in, D->y_d.p, D->ld_out, B, g_stream);
  if (!rc && copies) {
    hipError_t e = hipMemcpyAsync(D->pin_out.p, D->y_d.p, (size_t)B * D->ld_out * es, hipMemcpyDeviceToHost,
                                  g_stream);
    if (e != hipSuccess) rc = kans_fail(KANS_ERR_HIP, "capture D2H: %s", hipGetErrorString(e));
  }
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(g_stream, &g);
  if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
  if (e != hipSuccess) return kans_fail(KANS_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
  D->graph = g;
  HIP_TRY(hipGraphInstantiate(&D->exec, D->graph, nullptr, nullptr, 0));
  D->graph_B = B;
  D->graph_in = D->in_dtype;
  D->graph_gen = dgated_gen(D);
  D->graph_copies = copies;
  return 0;
}

static int dgated_graph_ready(kans_gated_dense* D, int B, bool copies) {
  int rc = dgated_reserve(D, B);
  if (rc) return rc;
  if (D->exec && D->graph_B == B && D->graph_in == D->in_dtype && D->graph_gen == dgated_gen(D) &&
      D->graph_copies == copies)
    return 0;
  return dgated_capture(D, B, copies);
}

extern "C" {

int kans_gated_dense_create(kans_layer* gate, kans_layer* up, kans_layer* down, kans_gated_dense** out) {
  if (!gate || !up || !down || !out) return kans_fail(KANS_ERR_ARG, "null argument");
  if (gate->dtype != up->dtype || gate->dtype != down->dtype)
    return kans_fail(KANS_ERR_ARG, "gate, up and down must share one dtype");
  if (gate->D_in != up->D_in || gate->D_out != up->D_out || down->D_in != gate->D_out || down->D_out != gate->D_in)
    return kans_fail(KANS_ERR_ARG, "shape mismatch: gate %dx%d, up %dx%d, down %dx%d", gate->D_in, gate->D_out,
                     up->D_in, up->D_out, down->D_in, down->D_out);
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = ensure_init();
  if (rc) return rc;
  auto* D = new kans_gated_dense();
  D->gate = gate;
  D->up = up;
  D->down = down;
  D->dtype = gate->dtype;
  D->in_dtype = D->dtype;
  D->d = gate->D_in;
  D->h = gate->D_out;
  D->ld_in = gate->D_in8;
  D->ld_h = round_up(D->h, 8);
  D->ld_out = D->d;
  *out = D;
  return 0;
}

int kans_gated_dense_destroy(kans_gated_dense* D) {
  if (!D) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ready) (void)hipStreamSynchronize(g_stream);
  delete D;
  return 0;
}

// Device arrays: X [B][ldx] (x_dtype: the block dtype, or fp32 for a 16-bit block; ldx >= round_up(d, 8),
// a multiple of 8), Y [B][ldy] in the block dtype; eager launches on `stream`.
int kans_gated_dense_forward(kans_gated_dense* D, const void* X, int x_dtype, long ldx, void* Y, long ldy, int B,
                             void* stream) {
  if (!D || !X || !Y || B < 0) return kans_fail(KANS_ERR_ARG, "bad argument");
  if (x_dtype != D->dtype && x_dtype != DT_F32) return kans_fail(KANS_ERR_ARG, "x_dtype must be the block dtype or fp32");
  if (B == 0) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = dgated_reserve(D, B);
  if (rc) return rc;
  return dgated_launch(D, X, x_dtype, ldx, Y, ldy, B, stream ? (hipStream_t)stream : g_stream);
}

// Host arrays [B][d] (x_dtype: the block dtype, or fp32 for a 16-bit block) -> [B][d] (block dtype):
// one graph replay (one H2D and one D2H copy).
int kans_gated_dense_forward_host(kans_gated_dense* D, const void* X, int x_dtype, void* Y, int B) {
  if (!D || (B > 0 && (!X || !Y)) || B < 0) return kans_fail(KANS_ERR_ARG, "bad argument");
  if (x_dtype != D->dtype && x_dtype != DT_F32) return kans_fail(KANS_ERR_ARG, "x_dtype must be the block dtype or fp32");
  if (B == 0) return 0;
  std::lock_guard<std::mutex> lk(g_mu);
  D->in_dtype = x_dtype;
  // the kernels-only graph; the host arrays are staged around it (stage_in / stage_out)
  int rc = dgated_graph_ready(D, B, false);
  if (rc) return rc;
  const size_t es = dtype_size(D->dtype), xes = dtype_size(x_dtype);
  const size_t in_bytes = (size_t)B * D->ld_in * xes, out_bytes = (size_t)B * D->ld_out * es;
  const size_t row_in = (size_t)D->d * xes, pitch_in = (size_t)D->ld_in * xes;
  if (g_async) {  // per-call pinned buffers; the result lands in Y at metal_kan_sync
    void* pin_in;
    void* pin_out;
    HIP_TRY(hipHostMalloc(&pin_in, in_bytes, hipHostMallocDefault));
    if (hipHostMalloc(&pin_out, out_bytes, hipHostMallocDefault) != hipSuccess) {
      (void)hipHostFree(pin_in);
      return kans_fail(KANS_ERR_HIP, "hipHostMalloc of %zu bytes failed", out_bytes);
    }
    // both buffers are freed at the next sync; Y is registered only once every step is enqueued
    g_pending.push_back({pin_in, nullptr, 0});
    g_pending.push_back({pin_out, nullptr, 0});
    const size_t out_idx = g_pending.size() - 1;
    if ((rc = stage_in(D->x_d.p, X, row_in, pitch_in, B, pin_in, g_stream))) return rc;
    HIP_TRY(hipGraphLaunch(D->exec, g_stream));
    HIP_TRY(hipMemcpyAsync(pin_out, D->y_d.p, out_bytes, hipMemcpyDeviceToHost, g_stream));
    g_pending[out_idx].dst = Y;
    g_pending[out_idx].bytes = out_bytes;
    return 0;
  }
  if ((rc = stage_in(D->x_d.p, X, row_in, pitch_in, B, D->pin_in.p, g_stream))) return rc;
  if (hipGraphLaunch(D->exec, g_stream) != hipSuccess) {
    (void)hipStreamSynchronize(g_stream);  // the input DMAs read pin_in; finish them before it is reused
    return kans_fail(KANS_ERR_HIP, "hipGraphLaunch failed");
  }
  return stage_out(Y, D->y_d.p, out_bytes, D->pin_out.p, g_stream);
}

// Mean ms per graph replay on the block's device buffers (include_copies: with the pinned H2D / D2H copies;
// the input dtype of the last host call).
int kans_gated_dense_time(kans_gated_dense* D, int B, int warmup, int iters, int include_copies, float* ms) {
  if (!D || B <= 0 || iters <= 0 || !ms) return kans_fail(KANS_ERR_ARG, "bad argument");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = dgated_graph_ready(D, B, include_copies != 0);
  if (rc) return rc;
  for (int i = 0; i < warmup; ++i) HIP_TRY(hipGraphLaunch(D->exec, g_stream));
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0));
  HIP_TRY(hipEventCreate(&e1));
  HIP_TRY(hipEventRecord(e0, g_stream));
  for (int i = 0; i < iters; ++i) HIP_TRY(hipGraphLaunch(D->exec, g_stream));
  HIP_TRY(hipEventRecord(e1, g_stream));
  HIP_TRY(hipEventSynchronize(e1));
  float t = 0;
  HIP_TRY(hipEventElapsedTime(&t, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *ms = t / iters;
  return 0;
}

}  // extern "C"
