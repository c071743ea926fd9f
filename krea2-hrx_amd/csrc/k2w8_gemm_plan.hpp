// Which tile kernel a GEMM shape runs (launch_gemm), as pure host functions of the
// shape and the CU count, so the rule can be tested without a GPU. The few-token
// kernel is chosen before these (skinny_streams).
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace k2w8 {

enum class GemmTile : int {
  k256x256 = 0,  // eight waves (4 x 2), two stages; with n_big > 0, columns past n_big run as 128x128
  k256x192 = 1,  // eight waves, two stages
  k256x128 = 2,  // eight waves, two stages (two workgroups per CU)
  k256x128Deep = 3,  // eight waves, three stages (one workgroup per CU)
  k128x128 = 4,  // four waves, two stages
  k128x64 = 5,   // eight waves, three stages
  k64x64 = 6,    // two K groups of four waves, four stages
  kSplit = 7,    // split K over 128x128 tiles when the workspace allows it, else 64x64
};

struct TilePlan {
  GemmTile tile = GemmTile::k64x64;
  int64_t n_big = 0;  // k256x256 only: the columns that run as 256x256 tiles (0: all)
};

// A round of 128x128 tiles against a round of 256x256 ones (measured 27 us against
// 61 us at K=3072), in units of tile width.
constexpr int64_t kTailCost = 115;
// Fewest 128-byte K steps a split-K slice takes.
constexpr int64_t kSplitMinSteps = 4;

// Tile choice: 256x256 or 256x192 when they give at least a full round (or, for one
// round, half the CUs), by rounds x width; else 256x128 when it gives every CU a
// workgroup (three stages when it gives more than half of them one, for M > 128);
// 128x128 when it gives every CU a workgroup; 128x64, then 64x64, for K up to 4096;
// else split K (kSplit).
inline TilePlan plan_tiles(int64_t m, int64_t n, int64_t k, int64_t cus) {
  auto tiles = [&](int64_t bm, int64_t bn) { return ((m + bm - 1) / bm) * (n / bn); };
  auto rounds = [&](int64_t t) { return (t + cus - 1) / cus; };
  // Wide tiles. A tile's time is about proportional to its width, so the candidates
  // compare by rounds x width: 256x256 (whole rounds, the columns of a last, mostly
  // idle round re-tiled as one round of 128x128 tiles, about 0.45 of a 256x256 round),
  // or 256x192. Measured: QKV 4096x9216 144 -> 135 us, config 1 (4096x3072) 52 -> 46 us.
  int64_t cost256 = INT64_MAX, n_big = 0;
  if (n % 256 == 0 && (tiles(256, 256) >= cus || (tiles(256, 128) > cus && 2 * tiles(256, 256) >= cus))) {
    const int64_t tm = (m + 255) / 256, total = tm * (n / 256);
    cost256 = rounds(total) * 256;
    const int64_t rest = total % cus, nb = (total / cus) * cus / tm * 256;
    if (total >= cus && rest > 0 && rest * 2 <= cus && nb > 0 && nb < n &&
        ((m + 127) / 128) * ((n - nb) / 128) <= cus) {
      n_big = nb;
      cost256 = (total / cus) * 256 + kTailCost;
    }
  }
  if (cost256 != INT64_MAX) {
    // 256x192 tiles read 11% more LDS bytes per MFMA: they must win by 5%.
    if (n % 192 == 0 && 2 * tiles(256, 192) >= cus && rounds(tiles(256, 192)) * 192 * 21 < cost256 * 20)
      return TilePlan{GemmTile::k256x192, 0};
    return TilePlan{GemmTile::k256x256, n_big};
  }
  if (tiles(256, 128) >= cus) return TilePlan{GemmTile::k256x128, 0};
  // One round of 256x128 tiles over more than half the CUs: one workgroup per CU, so
  // three stages fit (two K steps in flight). SwiGLU-up at M=256: 34.6 -> 31.3 us
  // against 128x128 tiles.
  if (m > 128 && 2 * tiles(256, 128) > cus) return TilePlan{GemmTile::k256x128Deep, 0};
  if (tiles(128, 128) >= cus) return TilePlan{GemmTile::k128x128, 0};
  // 64x64 tiles read every operand byte 4x as often as 128x128 ones: past K=4096 the
  // split-K pass over 128x128 tiles moves fewer bytes.
  if (tiles(128, 64) >= cus && k <= 4096) return TilePlan{GemmTile::k128x64, 0};
  if (tiles(64, 64) >= cus && k <= 4096) return TilePlan{GemmTile::k64x64, 0};
  return TilePlan{GemmTile::kSplit, 0};
}

// Split K over 128x128 tiles when they would leave most CUs idle: enough slices to
// give every CU a workgroup, each at least kSplitMinSteps K steps, within the
// workspace. Returns the K steps per slice, or 0 for no split.
inline int splitk_steps(int64_t m, int64_t n, int64_t k, int64_t cus, size_t workspace_bytes) {
  const int64_t tiles = ((m + 127) / 128) * (n / 128);
  const int64_t k_steps = k / 128;
  if (tiles * 2 > cus || k_steps < 2 * kSplitMinSteps) return 0;
  // As many splits as keep the grid to one workgroup per CU (one round): a second,
  // partial round costs more than the K steps it takes off each slice.
  int64_t splits = cus / tiles;
  if (splits > k_steps / kSplitMinSteps) splits = k_steps / kSplitMinSteps;
  const int64_t slice_bytes = m * n * 4;
  if (slice_bytes >= (int64_t)1 << 31) return 0;  // buffer offsets within a slice are 32-bit
  const int64_t fit = (int64_t)(workspace_bytes / (size_t)slice_bytes);
  if (splits > fit) splits = fit;
  if (splits < 2) return 0;
  const int64_t per = (k_steps + splits - 1) / splits;
  return (k_steps + per - 1) / per >= 2 ? (int)per : 0;
}

// A call whose workspace is fixed and required (the allocation-free entry point): a
// shape that would split K with an unbounded workspace but whose two slices do not fit
// the fixed one is refused, rather than run on the slower 64x64 tiles.
inline bool splitk_refused(int64_t m, int64_t n, int64_t k, int64_t cus, size_t workspace_bytes) {
  return plan_tiles(m, n, k, cus).tile == GemmTile::kSplit && splitk_steps(m, n, k, cus, SIZE_MAX) > 0 &&
         (size_t)(2 * m * n * 4) > workspace_bytes;
}

// Whether a prepare -> GEMM pair can run as the one persistent launch (one workgroup
// per CU, all resident): whole rounds of 256x192 tiles, rows the prepare writes at the
// stride the GEMM reads, and a row of at most 3072 (the prepare phase's registers).
inline bool one_launch_fits(int64_t tokens, int64_t m, int64_t n, int64_t width, int64_t lda,
                            int64_t out_stride, int64_t cus) {
  if (width > 3072 || m != tokens || lda != out_stride || n % 192 != 0 || cus < 1) return false;
  return ((m + 255) / 256) * (n / 192) % cus == 0;
}

}  // namespace k2w8
