// Launchers of the five GEMV layouts, compiled in their own sources
// (gemv_block.hip: layout 0; gemv_wave.hip: layout 1; gemv_mfma.hip: layouts 2,
// 3 and 4) and called
// by the C entry points in gemv.hip, plus the shape rules those entry points
// validate against.
#pragma once

#include "gemv_core.h"

namespace ko {

constexpr int LDS_X_BYTES = 40960;  // layout 1: normalised x staged for the workgroup (M*K*2)
constexpr int MFMA_CUS = 256;       // MI355X compute units: layout-2 grid of at most 256 x rows
constexpr int KS_MAX = 32;          // layout 3: slices per tile
constexpr int SK_W = 10;            // layout 4: wavefronts (chunks) per workgroup
constexpr int SK_CPT = 16;          // layout 4: chunks per tile
constexpr int SK_SPT = 3;           // layout 4: workgroups a tile's chunks can span (SK_W < SK_CPT)

// layout 0: `rows` (4, 8; 16 for M <= 2) columns per 256-thread workgroup
int launch_layout0(const GemvArgs& a, int epi, bool norm, int rows, hipStream_t s);
// layout 1: `rw` columns per wavefront, `wpb` wavefronts per workgroup
int launch_layout1(const GemvArgs& a, int epi, bool norm, int rw, int wpb, hipStream_t s);
// layout 2: MFMA tiles, a persistent grid of at most MFMA_CUS * per_cu workgroups;
// mt row tiles of 16 rows of x per weight pass (1, or 2 for K <= 4096)
int launch_layout2(const GemvArgs& a, int epi, bool norm, int per_cu, int mt, hipStream_t s);
// layout 3: MFMA tiles with the K range cut into `slices`
int launch_layout3(const GemvArgs& a, int epi, bool norm, int slices, int* ctr, float* slots,
                   hipStream_t s);
// layout 4: MFMA tiles cut into SK_CPT chunks dealt out SK_W per workgroup
// layout 4: stream-K over the tiles' K chunks; mt row tiles of 16 rows of x per weight pass
int launch_layout4(const GemvArgs& a, int epi, int mt, int* ctr, float* slots, hipStream_t s);

// Workgroups of the layout-2 grid: at most MFMA_CUS * per_cu, and of those the
// fewest that keep the most tiles per workgroup at its minimum, so every
// workgroup runs the same number of tiles (but the last ones, one fewer). A
// part-filled last round leaves the busy workgroups as long as the full ones
// and only spreads the weights over more CUs: 16 rows, 384 tiles on 192
// workgroups 10.14 against 10.52 us on 256; 608 tiles on 203 workgroups 19.85
// against 20.70 us.
inline int mfma_grid(int N, int per_cu) {
  const int ntiles = (N + 15) / 16;
  const int g = MFMA_CUS * per_cu;
  if (ntiles <= g) return ntiles;
  const int rounds = (ntiles + g - 1) / g;
  return (ntiles + rounds - 1) / rounds;
}

// K = 32 * S * WPG: S steps of 32 per wavefront, WPG wavefronts splitting K.
// SWIGLU (two weight tiles) needs K <= 4096 to keep its registers; 32 rows
// (two row tiles of x) need K <= 4096, SWIGLU K = 2560.
inline bool mfma_supported(int K, int epi, int mt = 1) {
  if (mt == 2) return K == 2560 || (K == 4096 && epi != EPI_SWIGLU);
  return K == 2560 || K == 4096 || (K == 9728 && epi != EPI_SWIGLU);
}

// Rows of x per launch of a layout: 4 (layout 1), 32 (layouts 2 and 4 with two
// row tiles, waves == 2), 64 (layout 4 with four, waves == 4), else 16.
inline int mstep_for(int layout, int waves) {
  if (layout == 1) return 4;
  if ((layout == 2 || layout == 4) && waves == 2) return 32;
  if (layout == 4 && waves == 4) return 64;
  return 16;
}
// Row tiles of a launch slice of mr rows under a layout-4 `waves` (0, 2 or 4):
// the fewest that hold the slice.
inline int sk_tiles(int waves, int mr) {
  if (waves == 0) return 1;
  return mr > 32 && waves == 4 ? 4 : mr > 16 ? 2 : 1;
}

// Steps per wavefront of layout 3 for K and a slice count (0: unsupported):
// S in {20, 19, 8, 4} with K = 128 * S * slices.
inline int ks_steps(int K, int slices) {
  if (slices < 1 || slices > KS_MAX || K % (128 * slices)) return 0;
  const int S = K / (128 * slices);
  return (S == 20 || S == 19 || S == 8 || S == 4) ? S : 0;
}

// Layout 3 scratch (fp32 elements): the tiles' arrival counters (int32, zero
// before the first launch, left at zero by every launch), padded to 64, then
// two 16 x 16 fp32 slots (gate and up) per (tile, slice).
inline long long ks_scratch(int N, int slices) {
  const long long T = (N + 15) / 16;
  return ((T + 63) / 64) * 64 + T * slices * 2 * 256;
}

// Layout 4: steps per chunk (K = 512 S; 0: unsupported), the grid, and the
// scratch (fp32 elements): the tiles' arrival counters as in layout 3, then
// SK_SPT 16 x 16 fp32 slots per tile.
inline int sk_steps(int K) {
  if (K % (32 * SK_CPT)) return 0;
  const int S = K / (32 * SK_CPT);
  return (S == 19 || S == 8 || S == 5) ? S : 0;
}
inline int sk_grid(int N) { return ((N + 15) / 16 * SK_CPT + SK_W - 1) / SK_W; }
// layout 4's scratch: the tiles' arrival counters (padded to 64), then each
// tile's SK_SPT slots of mt * 256 floats (mt row tiles of 16 x 16)
inline long long sk_scratch(int N, int mt = 1) {
  const long long T = (N + 15) / 16;
  return ((T + 63) / 64) * 64 + T * SK_SPT * 256 * mt;
}

}  // namespace ko
