// tiles.hpp - the gfx950 GEMM tile table of libjules_hip (internal).
//
// One table decides which kernel, and so which workgroup tile, every GEMM
// launch uses.  The launchers (gemm_f32.hip, gemm_bf16.hip) read it, and so
// does jules::kernel::TilePlanner (kernel_shims.cpp), whose getTileConfig
// therefore returns the tile that actually runs (the reference's planner,
// TilePlanner.h:74-136, sizes tiles for the CPU caches instead).
//
// fp32 (the bit-exact fma-chain GEMM): every variant computes each output as
// the same sequential fma chain over k, so the choice changes speed, never
// bits.  The variants:
//   F32_ROWS1 / F32_ROWS2: a wave owns 1 or 2 rows x 64 columns, 4 waves per
//     workgroup; the workgroup's rows of A (all of K) sit in LDS, so K is
//     limited to kF32RowsMaxK, and B streams through an LDS ring by LDS DMA.
//     Tile (4*rw) x 64 x K.
//   F32_T32 / F32_T64: 32x32 (2x2 per thread) and 64x64 (4x4 per thread)
//     output tiles, A and B staged through LDS in K slices of 32.
// bf16 (MFMA): 256x256 output tiles of 4 waves; BF16_DMA copies 32-deep K
// slices HBM -> LDS with LDS DMA (full tiles only), BF16_REG stages 64-deep
// slices through registers and zero-fills ragged edges.
#pragma once

#include <stdint.h>

namespace jh {

enum GemmVariant {
    GV_F32_ROWS1 = 0,
    GV_F32_ROWS2 = 1,
    GV_F32_T32 = 2,
    GV_F32_T64 = 3,
    GV_BF16_DMA = 4,
    GV_BF16_REG = 5,
    GV_COUNT = 6
};

struct GemmTile {
    int variant;
    int tile_m;
    int tile_n;
    int tile_k;
};

constexpr int kF32RowsWaves = 4;     // waves per row-kernel workgroup
constexpr int kF32RowsMaxK = 2048;   // 2 rows x 4 waves x K floats of A in 64 KiB of LDS
constexpr int kF32SliceK = 32;       // K slice of the LDS-tiled fp32 kernels
constexpr int kBf16Tile = 256;       // bf16 output tile (both variants)
constexpr int kBf16DmaK = 32;        // k per LDS-DMA stage
constexpr int kBf16RegK = 64;        // k per register-staged slice

inline bool f32_variant_valid(int v, int K) {
    if (v == GV_F32_ROWS1 || v == GV_F32_ROWS2) return K <= kF32RowsMaxK;
    return v == GV_F32_T32 || v == GV_F32_T64;
}

inline GemmTile f32_variant_tile(int v, int K) {
    switch (v) {
    case GV_F32_ROWS1: return {v, kF32RowsWaves, 64, (K + 3) & ~3};
    case GV_F32_ROWS2: return {v, 2 * kF32RowsWaves, 64, (K + 3) & ~3};
    case GV_F32_T32: return {v, 32, 32, kF32SliceK};
    default: return {GV_F32_T64, 64, 64, kF32SliceK};
    }
}

// The variant an fp32 GEMM launch uses.  Up to 1M outputs (and K within the
// row kernel's LDS): the row kernel, 2 rows per wave, or 1 when 2 would
// leave fewer than 1024 waves (512^3: 21.7 us at 2 rows, 27.1 us at 1;
// 64x256x784: 20.4 us at 1 row, 23.6 us at 2).  Larger: 64x64 tiles once
// there are at least 512 of them (two per CU), else 32x32.
inline GemmTile f32_gemm_tile(int M, int N, int K) {
    if ((int64_t)M * N <= (int64_t(1) << 20) && K <= kF32RowsMaxK) {
        const bool one = (((int64_t)N + 63) / 64) * (((int64_t)M + 1) / 2) < 1024;
        return f32_variant_tile(one ? GV_F32_ROWS1 : GV_F32_ROWS2, K);
    }
    const int64_t tiles64 = (((int64_t)M + 63) / 64) * (((int64_t)N + 63) / 64);
    return f32_variant_tile(tiles64 >= 512 ? GV_F32_T64 : GV_F32_T32, K);
}

// The variant a bf16 GEMM launch uses: LDS DMA when M and N are multiples of
// the 256 tile and K of the 32-deep stage, register staging otherwise.
inline GemmTile bf16_gemm_tile(int M, int N, int K) {
    const bool full = M % kBf16Tile == 0 && N % kBf16Tile == 0 && K % kBf16DmaK == 0 && K > 0;
    return full ? GemmTile{GV_BF16_DMA, kBf16Tile, kBf16Tile, kBf16DmaK}
                : GemmTile{GV_BF16_REG, kBf16Tile, kBf16Tile, kBf16RegK};
}

}  // namespace jh
