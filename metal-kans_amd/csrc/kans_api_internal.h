// Internal declarations shared by the runtime and kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include "kans_common.h"
#include "../../include/kans_hip.h"
#include <mutex>
#include <vector>

namespace kans {

// One fused dense launch (see kans_dense.hip).
struct DenseLaunch {
  int dtype, basis, has_base;
  int x_dtype, y_dtype;  // element types of X and Y: dtype, or DT_F32
  const void* X; long ldx;
  const void* Wt; int nob_pad;
  const void* bias;
  void* Y; long ldy;
  float* part;          // split workspace (splits * B * D_out floats) or null
  int B, D_in, D_out, nfb;
  BasisParams bp;
  int wm, nb, splits;   // tile config
  int ks = 1;           // wave groups per workgroup (4-wave block kernel, block_wave_groups_ok)
  int pair = 1;         // block kernels: two feature blocks per LDS stage when they fit (kan_fused_block)
};

// RBF parameters (centres, scaled centres, recurrence eligibility) of bp (bp.K set) from K centres and
// inv_denominator = 1/(2h^2); false (bp unchanged) when inv_den is negative or not finite
// (kans_runtime.hip).
bool kans_set_rbf_params(BasisParams& bp, const float* centers, float inv_den);

// Host <-> device staging through pinned memory, the host copies split over worker threads and
// overlapped with the DMAs (kans_staging.hip; call with the library lock held).
// stage_in: `rows` rows of `row_bytes` bytes, contiguous in host src, into device rows of `pitch` bytes
// (the tail of each row zeroed) through the pinned buffer `pin` (>= rows * pitch bytes).  Returns once
// every DMA is enqueued on st; `pin` stays in use until st has passed them.
int stage_in(void* dst, const void* src, size_t row_bytes, size_t pitch, long rows, void* pin, hipStream_t st);
// stage_out: `bytes` from device src, after the work already on st, into host dst through the pinned
// buffer `pin` (>= bytes).  Returns when dst holds them.
int stage_out(void* dst, const void* src, size_t bytes, void* pin, hipStream_t st);
// The same in two parts, for transfers from several streams: stage_out_enqueue adds the device -> pinned
// copies of one range (after the work already on st) to `out`; stage_out_drain waits for the pieces in
// the order they were added and copies each into host memory as it lands.
struct StagedOut {
  struct Piece {
    char* dst;
    const char* pin;
    size_t bytes;
  };
  std::vector<Piece> pieces;
  size_t bytes = 0;
};
int stage_out_enqueue(StagedOut& out, void* dst, const void* src, size_t bytes, void* pin, hipStream_t st);
int stage_out_drain(StagedOut& out);

}  // namespace kans

int kans_fail(int code, const char* fmt, ...);
// Per-device set-up of kans_gated_forward_noalloc's scratch (kans_qruntime.hip);
// called by the library's initialisation with `device` current.
int kans_noalloc_setup(int device);
hipStream_t kans_default_stream();
// fp32 Chebyshev forward (no base branch) of host X on device-resident fp32 weights (kans_runtime.hip);
// call with the library lock held.
int kans_ref_cheby_forward_devw_locked(const float* X, const float* W_dev, const float* bias_dev, float* Y, int B,
                                       int D_in, int D_out, int K, int has_bias);

// Library lock (serialises every entry point that touches device state), lazy
// device initialisation (call with the lock held) and the grow-only pinned
// staging buffers of the synchronous host-pointer entry points (which = 0 in,
// 1 out; lock held).
std::mutex& kans_mutex();
int kans_ensure_init();
int kans_pinned_stage(int which, size_t bytes, void** p);

#define HIP_TRY(expr)                                                                       \
  do {                                                                                      \
    hipError_t _e = (expr);                                                                 \
    if (_e != hipSuccess)                                                                   \
      return kans_fail(KANS_ERR_HIP, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), \
                       __FILE__, __LINE__);                                                 \
  } while (0)

// Grow-only device buffer.
struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { if (p) (void)hipFree(p); }
  int reserve(size_t bytes) {
    if (bytes <= cap) return 0;
    if (p) HIP_TRY(hipFree(p));
    p = nullptr;
    cap = 0;
    HIP_TRY(hipMalloc(&p, bytes));
    cap = bytes;
    return 0;
  }
};

// Grow-only pinned host buffer.
struct Pinned {
  void* p = nullptr;
  size_t cap = 0;
};
inline int pinned_reserve(Pinned& b, size_t bytes) {
  if (bytes <= b.cap) return 0;
  if (b.p) HIP_TRY(hipHostFree(b.p));
  b.p = nullptr;
  b.cap = 0;
  size_t cap = bytes + bytes / 4;
  HIP_TRY(hipHostMalloc(&b.p, cap, hipHostMallocDefault));
  b.cap = cap;
  return 0;
}
