// Host <-> device staging of the synchronous host-pointer entry points.
//
// A host array reaches the device through a pinned buffer (the caller's own
// memory is never registered).  Copying a whole array into the pinned buffer
// on one thread, then one DMA, the kernels, one DMA back and one copy out on
// one thread again costs far more than the kernels at large batches: at the
// 16384 x 1024 fp16 shape (33.5 MB each way) a call took 5.1 ms around a
// 0.28 ms kernel, most of it the two host copies (the copy into a caller's
// freshly allocated output array is dominated by first-touch page faults).
//
// Here each transfer is cut into pieces of about kPieceBytes.  Up to
// kStageThreads worker threads copy pieces in parallel (page faults included),
// claiming them in increasing order.  Input: the calling thread issues each
// piece's DMA as soon as that piece is in pinned memory, so the host copies
// overlap the DMAs.  Output: the calling thread enqueues every piece's DMA with
// an event behind it, then releases each piece to the workers as soon as its
// event has completed.  Every HIP call is made by the calling thread, which
// holds the library lock; the calling thread also copies pieces whenever it
// would otherwise wait, so the transfer completes even if no worker thread
// could be started.  Transfers below kThreadedBytes take one copy and one DMA.
//
// The caller's output array is often freshly allocated (numpy's np.empty of a
// large array is a fresh anonymous mapping), so the output copy spends most of
// its time in first-touch page faults.  stage_out asks for transparent huge
// pages on the page-aligned interior of the output first (madvise, a hint: it
// changes no contents and is ignored for file-backed memory or where the
// system disables them) and copies with up to kStageOutThreads threads.
// Measured on the GPU box (16 CPUs, THP in madvise mode), 33.5 MB from pinned
// memory into freshly malloc'ed memory: 4 threads 2.8 ms, with the hint 1.1 ms;
// 8 threads 1.5 / 1.0 ms.  Copies into pinned memory saturate at 4 threads
// (0.44 ms for 33.5 MB).
#include "kans_api_internal.h"

#include <sched.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstring>
#include <memory>
#include <system_error>
#include <thread>
#include <vector>

namespace kans {
namespace {

constexpr size_t kPieceBytes = size_t(2) << 20;
constexpr size_t kThreadedBytes = size_t(4) << 20;
constexpr int kStageThreads = 4;
constexpr int kStageOutThreads = 8;

// CPUs this process may run on (its affinity mask), at least 1.
int cpu_share() {
  static const int n = [] {
    cpu_set_t set;
    CPU_ZERO(&set);
    if (sched_getaffinity(0, sizeof set, &set) == 0 && CPU_COUNT(&set) > 0) return (int)CPU_COUNT(&set);
    const unsigned h = std::thread::hardware_concurrency();
    return h > 0 ? (int)h : 1;
  }();
  return n;
}

// Worker threads for a transfer of n pieces: at most `cap`, at most one per piece, and leaving half of
// the process's CPUs to the rest of the program.
int workers_for(int n, int cap) { return std::max(1, std::min({cap, n, cpu_share() / 2})); }

void hint_huge_pages(void* dst, size_t bytes) {
  const long pg = sysconf(_SC_PAGESIZE);
  if (pg <= 0) return;
  const uintptr_t a = ((uintptr_t)dst + (uintptr_t)pg - 1) & ~((uintptr_t)pg - 1);
  const uintptr_t e = ((uintptr_t)dst + bytes) & ~((uintptr_t)pg - 1);
  if (e > a) (void)madvise((void*)a, e - a, MADV_HUGEPAGE);
}

// Pieces of `rows` rows of `pitch` bytes: piece k is rows [r0(k), r1(k)).
struct Pieces {
  long rows, rpp;
  int n;
  Pieces(long rows_, size_t pitch)
      : rows(rows_), rpp(std::max<long>(1, (long)(kPieceBytes / std::max<size_t>(pitch, 1)))) {
    n = (int)((rows + rpp - 1) / rpp);
  }
  long r0(int k) const { return (long)k * rpp; }
  long r1(int k) const { return std::min(rows, (long)(k + 1) * rpp); }
};

// Rows [r0, r1) of src (row_bytes each, contiguous) into pinned rows of pitch bytes, the tail of each
// pinned row zeroed.
void copy_rows_in(char* pin, const char* src, size_t row_bytes, size_t pitch, long r0, long r1) {
  if (pitch == row_bytes) {
    memcpy(pin + (size_t)r0 * pitch, src + (size_t)r0 * row_bytes, (size_t)(r1 - r0) * pitch);
    return;
  }
  for (long r = r0; r < r1; ++r) {
    memcpy(pin + (size_t)r * pitch, src + (size_t)r * row_bytes, row_bytes);
    memset(pin + (size_t)r * pitch + row_bytes, 0, pitch - row_bytes);
  }
}

// Starts up to `want` threads running `body`; fewer if the system refuses more.
template <typename F>
void start_workers(std::vector<std::thread>& th, int want, F&& body) {
  th.reserve(want);
  for (int t = 0; t < want; ++t) {
    try {
      th.emplace_back(body);
    } catch (const std::system_error&) {
      break;
    }
  }
}

// Events of the output pieces (grow-only; the library lock guards them).
std::vector<hipEvent_t> g_piece_events;

int piece_events(int n) {
  while ((int)g_piece_events.size() < n) {
    hipEvent_t e;
    HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    g_piece_events.push_back(e);
  }
  return 0;
}

}  // namespace

int stage_in(void* dst, const void* src, size_t row_bytes, size_t pitch, long rows, void* pin, hipStream_t st) {
  if (rows <= 0) return 0;
  if (pitch < row_bytes) return kans_fail(KANS_ERR_ARG, "stage_in: pitch %zu < row bytes %zu", pitch, row_bytes);
  char* p = (char*)pin;
  char* d = (char*)dst;
  const char* s = (const char*)src;
  const size_t total = (size_t)rows * pitch;
  if (total < kThreadedBytes) {
    copy_rows_in(p, s, row_bytes, pitch, 0, rows);
    HIP_TRY(hipMemcpyAsync(d, p, total, hipMemcpyHostToDevice, st));
    return 0;
  }
  const Pieces P(rows, pitch);
  std::unique_ptr<std::atomic<int>[]> done(new std::atomic<int>[P.n]);
  for (int k = 0; k < P.n; ++k) done[k].store(0, std::memory_order_relaxed);
  std::atomic<int> next{0};
  auto copy_piece = [&](int k) {
    copy_rows_in(p, s, row_bytes, pitch, P.r0(k), P.r1(k));
    done[k].store(1, std::memory_order_release);
  };
  std::vector<std::thread> th;
  start_workers(th, workers_for(P.n, kStageThreads), [&] {
    for (int k; (k = next.fetch_add(1)) < P.n;) copy_piece(k);
  });
  hipError_t err = hipSuccess;
  for (int k = 0; k < P.n; ++k) {
    while (!done[k].load(std::memory_order_acquire)) {
      const int j = next.fetch_add(1);
      if (j < P.n) copy_piece(j);
      else std::this_thread::yield();
    }
    if (err == hipSuccess) {
      const size_t off = (size_t)P.r0(k) * pitch;
      err = hipMemcpyAsync(d + off, p + off, (size_t)(P.r1(k) - P.r0(k)) * pitch, hipMemcpyHostToDevice, st);
    }
  }
  for (auto& t : th) t.join();
  if (err != hipSuccess) {
    (void)hipStreamSynchronize(st);  // earlier pieces' DMAs still read pin
    return kans_fail(KANS_ERR_HIP, "hipMemcpyAsync of a staged input piece failed: %s", hipGetErrorString(err));
  }
  return 0;
}

int stage_out_enqueue(StagedOut& out, void* dst, const void* src, size_t bytes, void* pin, hipStream_t st) {
  if (bytes == 0) return 0;
  char* p = (char*)pin;
  char* d = (char*)dst;
  const char* s = (const char*)src;
  const Pieces P((long)bytes, 1);  // one-byte rows: pieces of kPieceBytes
  const int base = (int)out.pieces.size();
  int rc = piece_events(base + P.n);
  if (rc) return rc;
  if (bytes >= kThreadedBytes) hint_huge_pages(d, bytes);
  out.bytes += bytes;
  for (int k = 0; k < P.n; ++k) {
    const size_t len = (size_t)(P.r1(k) - P.r0(k));
    hipError_t e = hipMemcpyAsync(p + P.r0(k), s + P.r0(k), len, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipEventRecord(g_piece_events[base + k], st);
    if (e != hipSuccess) {
      (void)hipStreamSynchronize(st);
      return kans_fail(KANS_ERR_HIP, "enqueueing a staged output piece failed: %s", hipGetErrorString(e));
    }
    out.pieces.push_back({d + P.r0(k), p + P.r0(k), len});
  }
  return 0;
}

int stage_out_drain(StagedOut& out) {
  const int n = (int)out.pieces.size();
  if (n == 0) return 0;
  if (out.bytes < kThreadedBytes) {  // small: wait for everything, one copy per piece
    hipError_t e = hipSuccess;
    for (int k = 0; k < n && e == hipSuccess; ++k) e = hipEventSynchronize(g_piece_events[k]);
    if (e != hipSuccess) return kans_fail(KANS_ERR_HIP, "hipEventSynchronize: %s", hipGetErrorString(e));
    for (const auto& pc : out.pieces) memcpy(pc.dst, pc.pin, pc.bytes);
    out.pieces.clear();
    out.bytes = 0;
    return 0;
  }
  // ready[k]: 0 in flight, 1 in pinned memory, 2 abandoned (an event wait failed)
  std::unique_ptr<std::atomic<int>[]> ready(new std::atomic<int>[n]);
  for (int k = 0; k < n; ++k) ready[k].store(0, std::memory_order_relaxed);
  std::atomic<int> next{0};
  auto drain = [&] {
    for (int k; (k = next.fetch_add(1)) < n;) {
      int r;
      while ((r = ready[k].load(std::memory_order_acquire)) == 0) std::this_thread::yield();
      if (r != 1) continue;
      memcpy(out.pieces[k].dst, out.pieces[k].pin, out.pieces[k].bytes);
    }
  };
  std::vector<std::thread> th;
  start_workers(th, workers_for(n, kStageOutThreads), drain);
  hipError_t err = hipSuccess;
  for (int k = 0; k < n; ++k) {
    if (err == hipSuccess) err = hipEventSynchronize(g_piece_events[k]);
    ready[k].store(err == hipSuccess ? 1 : 2, std::memory_order_release);
  }
  drain();  // the calling thread copies whatever pieces are still unclaimed
  for (auto& t : th) t.join();
  out.pieces.clear();
  out.bytes = 0;
  if (err != hipSuccess) {
    (void)hipDeviceSynchronize();  // the pieces' streams may still write the pinned buffer
    return kans_fail(KANS_ERR_HIP, "hipEventSynchronize on a staged output piece failed: %s", hipGetErrorString(err));
  }
  return 0;
}

int stage_out(void* dst, const void* src, size_t bytes, void* pin, hipStream_t st) {
  if (bytes == 0) return 0;
  if (bytes < kThreadedBytes) {
    HIP_TRY(hipMemcpyAsync(pin, src, bytes, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    memcpy(dst, pin, bytes);
    return 0;
  }
  StagedOut out;
  int rc = stage_out_enqueue(out, dst, src, bytes, pin, st);
  if (rc) return rc;
  return stage_out_drain(out);
}

}  // namespace kans
