// Tile helpers shared by the fused dense kernels (kans_dense.hip) and the
// fused quantized-weight kernels (kans_qprefill_kernel.h): the 16-bit MFMA
// wrappers, the XCD-aware workgroup -> tile mapping and compile-time loops.
#pragma once
#include "kans_common.h"
#include <type_traits>

namespace kans {

template <typename T> struct Mfma;
template <> struct Mfma<_Float16> {
  typedef half8 frag;
  static __device__ __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<__bf16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ floatx16 mma(frag a, frag b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

// Remap the linear workgroup id so that consecutive ids of one XCD (the hardware
// deals workgroups round-robin over 8 XCDs) cover neighbouring tiles that share
// the same weight N-tile; keeps each XCD's L2 working on one slice of W'.
__device__ __forceinline__ int xcd_remap(int id, int total) {
  if ((total & 7) != 0) return id;
  int per = total >> 3;
  return (id & 7) * per + (id >> 3);
}

// Tile of linear index `lin` (after xcd_remap): tiles are visited in groups of
// GM m-tiles x all n-tiles, m fastest, so the 1/8 of the grid one XCD owns is a
// GM x (n_tiles/8)-ish block: its workgroups share input rows (x) and weight
// N-tiles (W') in that XCD's L2.
__device__ __forceinline__ void tile_of(int lin, int m_tiles, int n_tiles, int& m_tile, int& n_tile) {
  constexpr int GM = 16;
  const int group = lin / (GM * n_tiles);
  const int first_m = group * GM;
  const int gm = min(GM, m_tiles - first_m);
  const int in = lin - group * GM * n_tiles;
  m_tile = first_m + in % gm;
  n_tile = in / gm;
}

// Per-lane uint4 chunks of one 32-column block for element type T.
template <typename T> struct Chunks { static constexpr int CPL = (8 * (int)sizeof(T)) / 16; };

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

}  // namespace kans
