// sfg_gemm.hip -- projection / expert GEMMs for gfx950.
//
// Semantics: C[m][n] = sum_k A[m][k] * B[n][k] (B is the transposed, packed
// weight), fp32 accumulation, fused epilogues.  This replaces execute(LoopIR)
// (runtime.cpp:581-626), the MoE expert loops (moe_compiler.cpp:64-155) and
// weight-only int8 quantized_invoke (next_milestones.cpp:50-69).
//
// Kernels, picked by shape:
//  * gemm_skinny_kernel   M <= 64 rows (decode; grouped experts loop over
//    16- to 64-row passes): weight-streaming, HBM bound.
//    v_mfma_f32_16x16x32_bf16 with the activation rows as the A operand; bf16
//    or int8 weights (int8 -> bf16 is exact), 64 B contiguous per lane per
//    128-k chunk, split-K over up to 8 waves of one workgroup with a
//    fixed-order LDS reduction.
//  * gemm_splitk_kernel   33..64 dense rows with a caller workspace: 512-k
//    slices, activations staged once per workgroup in LDS, fp32 partials
//    summed in slice order by gemm_splitk_reduce_kernel (scale + epilogue).
//  * gemm_dma_kernel      bf16 prefill and grouped experts, >= 1024 rows:
//    256x256 (64-k slabs), 256x128, 128x256 or 128x128 tiles, operands global
//    -> LDS by DMA, v_mfma_f32_32x32x16_bf16, optional A-row gather and
//    per-group (expert) segments read from device offsets.
//  * gemm_mfma256_kernel  int8-weight products with >= 1024 rows: 256x128
//    tiles, k-slabs through padded LDS with register prefetch.
//  * gemm_mfma_kernel     the other tiled products (fewer rows, ragged N):
//    128x128x32 tiles through padded LDS with register prefetch.
//  * gemm_vec_kernel      fp32 operands (the fp32 configurations) and the
//    bf16 / int8 products the MFMA kernels do not lower: one sequential fp32
//    FMA chain per output on the VALU.
#include <type_traits>

#include "sfg_kernels.hpp"

#include <cstdlib>
#include <cstring>

namespace sfg {

namespace {

template <int EPI>
struct EpiTraits {
    static constexpr bool glu = (EPI == SFG_EPI_SWIGLU || EPI == SFG_EPI_GLU_SILU_UP);
};

__device__ __forceinline__ float glu_combine(int epi, float g, float u) {
    return epi == SFG_EPI_SWIGLU ? silu(g) * u : g * silu(u);
}

__device__ __forceinline__ void store_out(void* c, int c_dtype, int64_t idx, float v) {
    if (c_dtype == SFG_F32) static_cast<float*>(c)[idx] = v;
    else static_cast<uint16_t*>(c)[idx] = f32_to_bf16(v);
}

}  // namespace

// ===========================================================================
// Skinny (decode) GEMM.
//
// A workgroup owns NBT 16-row tiles of B (16 or 32 output columns; for GLU
// epilogues NBT / 2 gate tiles and the matching up tiles) and ALL of K: its WAVES
// waves split K into contiguous chunk ranges and reduce through LDS in a fixed
// order, so no workgroup waits for or publishes to another (no device-scope
// fences: on gfx950 they write back and invalidate the L2).  Each lane reads
// 64 B (bf16) / 32 B (int8) of one weight row per 128-k chunk.  A wave issues
// the loads of CB chunks (weights and activations) back to back before the
// first MFMA: loads retire in order, so interleaving prefetches with waits
// would expose the full memory latency on every chunk.
// ===========================================================================
struct SkinnyArgs {
    const uint16_t* a; int64_t lda; const int32_t* a_rows; int64_t a_rows_limit;
    const void* b; int64_t ldb; const float* scales;
    int64_t b_group_stride, s_group_stride;
    void* c; int c_dtype; int64_t ldc;
    const float* residual; int64_t ldr;
    int64_t m, n, k;
    const int32_t* offsets;
};

constexpr int kSkinnyChunk = 128;  // k per lane-chunk: 4 MFMA steps of 32
// Chunks whose loads a wave keeps in flight at once: what fits the register
// file at 8 waves per workgroup without spilling.
template <int MT>
constexpr int kSkinnyBatch = MT == 1 ? 4 : (MT == 2 ? 2 : 1);

template <int BDT, int MT, int NBT, int EPI, int WAVES, bool TILED>
__global__ __launch_bounds__(WAVES * 64) void gemm_skinny_kernel(SkinnyArgs p) {
    constexpr bool kGlu = EpiTraits<EPI>::glu;
    constexpr int CB = kSkinnyBatch<MT>;           // chunks in flight per wave
    constexpr int BQ = (BDT == SFG_I8) ? 2 : 4;    // uint4 per lane per chunk and tile
    static_assert(!kGlu || NBT == 2 || NBT == 4, "GLU epilogues pair gate and up tiles");
    constexpr int kGluTiles = NBT / 2;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = blockIdx.z;
    const int tile = blockIdx.x;
    int64_t rb = 0, re = p.m;
    if (p.offsets) {
        // Device-side bounds are data: clamp them so a corrupt table cannot
        // send the kernel outside [0, m).
        rb = min(max(static_cast<int64_t>(p.offsets[g]), int64_t(0)), p.m);
        re = min(max(static_cast<int64_t>(p.offsets[g + 1]), rb), p.m);
    }
    if (re <= rb) return;

    int64_t brow[NBT];
    int64_t out_col;
    if (kGlu) {
        out_col = static_cast<int64_t>(tile) * 16 * kGluTiles;
#pragma unroll
        for (int h = 0; h < kGluTiles; ++h) {
            brow[h] = out_col + 16 * h;                    // gate (or W1)
            brow[kGluTiles + h] = p.n + out_col + 16 * h;  // up (or W3)
        }
    } else {
        out_col = static_cast<int64_t>(tile) * (16 * NBT);
#pragma unroll
        for (int j = 0; j < NBT; ++j) brow[j] = out_col + 16 * j;
    }
    const int lr = lane & 15;   // A row / B column within a 16-tile
    const int lg = lane >> 4;   // k-group of the MFMA operand
    // MFMA k order is free as long as A and B agree.  bf16: step s of a chunk
    // reads k = 32 s + 8 lg + [0, 8), so the four lanes of a row read 64
    // contiguous bytes per instruction.  int8: a lane's 32 k are contiguous
    // (32 lg + 8 s + [0, 8)) and arrive as two 16-byte loads.
    constexpr int kLaneK = (BDT == SFG_I8) ? 32 : 8;
    constexpr int kStepK = (BDT == SFG_I8) ? 8 : 32;
    const char* bbase = static_cast<const char*>(p.b);
    const int64_t belem = (BDT == SFG_I8) ? 1 : 2;
    const int64_t bgroup = static_cast<int64_t>(g) * p.b_group_stride;
    const char* bptr[NBT];
    const int64_t chunk_count = p.k / kSkinnyChunk;
    constexpr int64_t kTileBytes = 16 * kSkinnyChunk * ((BDT == SFG_I8) ? 1 : 2);
#pragma unroll
    for (int j = 0; j < NBT; ++j) {
        if (TILED)  // fragment-tiled: tile (brow / 16, chunk) is kTileBytes contiguous
            bptr[j] = bbase + bgroup * belem + (brow[j] / 16) * chunk_count * kTileBytes + lane * 16;
        else
            bptr[j] = bbase + (bgroup + (brow[j] + lr) * p.ldb + lg * kLaneK) * belem;
    }
    const float* scales = p.scales ? p.scales + static_cast<int64_t>(g) * p.s_group_stride : nullptr;

    const int chunks = static_cast<int>(p.k / kSkinnyChunk);
    const int c_begin = chunks * wave / WAVES;
    const int c_end = chunks * (wave + 1) / WAVES;

    __shared__ floatx4 red[WAVES - 1][MT][NBT][64];

    for (int64_t pass = rb; pass < re; pass += MT * 16) {
        floatx4 acc[MT][NBT];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < NBT; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

        // Activation rows past the group or with a source index outside A
        // read row 0 instead (no branch around the loads): an MFMA output row
        // depends only on its own A row, and the epilogue stores nothing for
        // the former and the zero product for the latter.
        // 16-row blocks of this pass that hold rows (wave-uniform): a grouped
        // pass past its expert's rows skips the activation loads and MFMAs of
        // the empty blocks (their outputs are never stored)
        const int mt_live = static_cast<int>(min(static_cast<int64_t>(MT), (re - pass + 15) / 16));
        const uint16_t* arow[MT];
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const int64_t r = pass + i * 16 + lr;
            int64_t src = r < re ? (p.a_rows ? p.a_rows[r] : r) : 0;
            if (src < 0 || src >= p.a_rows_limit) src = 0;
            arow[i] = p.a + src * p.lda + lg * kLaneK;
        }

        for (int c0 = c_begin; c0 < c_end; c0 += CB) {
            uint4 bq[CB][NBT][BQ];
            uint4 aq[CB][MT][4];
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                if (c0 + c >= c_end) break;
                const int64_t kofs = static_cast<int64_t>(c0 + c) * kSkinnyChunk;
#pragma unroll
                for (int j = 0; j < NBT; ++j) {
                    if (TILED) {
                        // fragment s of this lane: 1 KB-contiguous wave loads
                        const char* pj = bptr[j] + static_cast<int64_t>(c0 + c) * kTileBytes;
#pragma unroll
                        for (int s = 0; s < BQ; ++s)
                            bq[c][j][s] = *reinterpret_cast<const uint4*>(pj + 1024 * s);
                    } else {
                        const char* pj = bptr[j] + kofs * belem;
#pragma unroll
                        for (int s = 0; s < BQ; ++s)
                            bq[c][j][s] = *reinterpret_cast<const uint4*>(
                                pj + (BDT == SFG_I8 ? 16 * s : 2 * kStepK * s));
                    }
                }
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    if (i > 0 && i >= mt_live) break;
                    const uint16_t* ap = arow[i] + kofs;
#pragma unroll
                    for (int s = 0; s < 4; ++s)
                        aq[c][i][s] = *reinterpret_cast<const uint4*>(ap + kStepK * s);
                }
            }
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                if (c0 + c >= c_end) break;
                bf16x8 bf[NBT][4];
#pragma unroll
                for (int j = 0; j < NBT; ++j) {
                    if (BDT == SFG_I8) {
                        bf[j][0] = as_bf16x8(i8x8_to_bf16x8(bq[c][j][0].x, bq[c][j][0].y));
                        bf[j][1] = as_bf16x8(i8x8_to_bf16x8(bq[c][j][0].z, bq[c][j][0].w));
                        bf[j][2] = as_bf16x8(i8x8_to_bf16x8(bq[c][j][1].x, bq[c][j][1].y));
                        bf[j][3] = as_bf16x8(i8x8_to_bf16x8(bq[c][j][1].z, bq[c][j][1].w));
                    } else {
#pragma unroll
                        for (int s = 0; s < 4; ++s) bf[j][s] = as_bf16x8(bq[c][j][s]);
                    }
                }
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    if (i > 0 && i >= mt_live) break;
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        const bf16x8 a = as_bf16x8(aq[c][i][s]);
#pragma unroll
                        for (int j = 0; j < NBT; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bf[j][s], acc[i][j], 0, 0, 0);
                    }
                }
            }
        }

        // Reduce the waves' partial sums in a fixed order (0 + 1 + ... ).
        if (wave > 0) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NBT; ++j) red[wave - 1][i][j][lane] = acc[i][j];
        }
        __syncthreads();
        if (wave == 0) {
            for (int w = 0; w < WAVES - 1; ++w)
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int j = 0; j < NBT; ++j) acc[i][j] += red[w][i][j][lane];
            // Everything the epilogue reads is loaded before its first store:
            // the output may alias these arrays for all the compiler knows,
            // so a load placed after a store would wait a full memory round
            // trip.  Rows past the group read its last row and store nothing.
            // Scale of B row brow[j] + lr (gate or up for GLU tiles).
            float sv[NBT];
            if (scales) {
#pragma unroll
                for (int j = 0; j < NBT; ++j) sv[j] = scales[brow[j] + lr];
            }
            float rv[MT][4][NBT];
            if constexpr (EPI == SFG_EPI_RESIDUAL && !kGlu) {
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int64_t row = min(pass + i * 16 + lg * 4 + r, re - 1);
#pragma unroll
                        for (int j = 0; j < NBT; ++j) rv[i][r][j] = p.residual[row * p.ldr + out_col + j * 16 + lr];
                    }
            }
            // gathered source indices: all loaded in one branch, compared after
            int32_t src_row[MT][4];
            if (p.a_rows) {
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) src_row[i][r] = p.a_rows[min(pass + i * 16 + lg * 4 + r, re - 1)];
            }
            bool zero_row[MT][4];
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    zero_row[i][r] = p.a_rows && (src_row[i][r] < 0 || src_row[i][r] >= p.a_rows_limit);
            // D layout: lane holds column (lane & 15), rows 4*(lane >> 4) + r.
#pragma unroll
            for (int i = 0; i < MT; ++i) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = pass + i * 16 + lg * 4 + r;
                    if (row >= re) continue;
                    // a gathered row whose source index is outside A multiplied zeros
                    if (zero_row[i][r]) {
#pragma unroll
                        for (int j = 0; j < NBT; ++j) acc[i][j][r] = 0.f;
                    }
                    if (kGlu) {
#pragma unroll
                        for (int h = 0; h < kGluTiles; ++h) {
                            const int64_t col = out_col + 16 * h + lr;
                            float gv = acc[i][h][r], uv = acc[i][kGluTiles + h][r];
                            if (scales) {
                                gv *= sv[h];
                                uv *= sv[kGluTiles + h];
                            }
                            store_out(p.c, p.c_dtype, row * p.ldc + col, glu_combine(EPI, gv, uv));
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < NBT; ++j) {
                            const int64_t col = out_col + j * 16 + lr;
                            float v = acc[i][j][r];
                            if (scales) v *= sv[j];
                            if constexpr (EPI == SFG_EPI_RESIDUAL) v += rv[i][r][j];
                            store_out(p.c, p.c_dtype, row * p.ldc + col, v);
                        }
                    }
                }
            }
        }
        __syncthreads();
    }
}

// ===========================================================================
// Split-K decode GEMM for 33..64 activation rows.
//
// With 64 rows the activations (64 x K bf16) outweigh the int8 weight slice a
// skinny workgroup streams, and a workgroup per 32 columns re-reads them from
// L2 for every column tile.  Here a workgroup owns 128 B rows (4 waves x two
// 16-row tiles) and one 512-k slice: it stages the slice's 64 activation rows
// in LDS once (rows padded by 16 B so the 16 rows of a fragment read fall on
// distinct banks), with every activation load and then every weight load of
// the slice in flight together (one memory round trip per workgroup), and
// writes raw fp32 partial sums [slice][m][n_b].  gemm_splitk_reduce_kernel
// then sums the slices in order 0, 1, ... and applies the per-channel scale
// and the epilogue, so the result does not depend on scheduling.
// ===========================================================================
struct SplitArgs {
    const uint16_t* a; int64_t lda;
    const void* b; int64_t ldb;
    float* part;   // [slices][m][nb]
    int64_t m, nb, k;
};

constexpr int kSplitKS = 512;                  // k per slice
constexpr int kSplitTiles = 2;                 // 16-row B tiles per wave
constexpr int kSplitCols = 64 * kSplitTiles;   // B rows per workgroup
constexpr int kSplitRows = 64;                 // activation rows staged
constexpr int kSplitLdA = kSplitKS + 8;        // bf16 per staged row
constexpr int kSplitChunks = kSplitKS / kSkinnyChunk;

template <int BDT, bool TILED>
__global__ __launch_bounds__(256) void gemm_splitk_kernel(SplitArgs p) {
    constexpr int BQ = (BDT == SFG_I8) ? 2 : 4;    // uint4 per lane per chunk and tile
    constexpr int kLaneK = (BDT == SFG_I8) ? 32 : 8;
    constexpr int kStepK = (BDT == SFG_I8) ? 8 : 32;
    __shared__ __attribute__((aligned(16))) uint16_t sa[kSplitRows * kSplitLdA];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int64_t k0 = static_cast<int64_t>(blockIdx.y) * kSplitKS;
    const int64_t col0 = static_cast<int64_t>(blockIdx.x) * kSplitCols + wave * 16 * kSplitTiles;

    // 1. the slice's activation rows, issued first:
    //    loads return in order, so their LDS stores wait on these alone
    constexpr int kVecsPerRow = kSplitKS / 8;
    constexpr int kStageVecs = kSplitRows * kVecsPerRow / 256;
    uint4 av[kStageVecs];
#pragma unroll
    for (int i = 0; i < kStageVecs; ++i) {
        const int q = tid + 256 * i;
        const int row = q / kVecsPerRow, v = q % kVecsPerRow;
        // rows past m read row m - 1 (no branch around the load: a
        // conditional load is waited for before the branches join) and are
        // zeroed at the store
        const int64_t src = row < p.m ? row : p.m - 1;
        av[i] = *reinterpret_cast<const uint4*>(p.a + src * p.lda + k0 + 8 * v);
    }
    // 2. every weight load of this wave's two tiles over the slice
    const char* bbase = static_cast<const char*>(p.b);
    const int64_t chunk_count = p.k / kSkinnyChunk;
    constexpr int64_t kTileBytes = 16 * kSkinnyChunk * ((BDT == SFG_I8) ? 1 : 2);
    uint4 bq[kSplitChunks][kSplitTiles][BQ];
#pragma unroll
    for (int j = 0; j < kSplitTiles; ++j) {
        const int64_t brow = col0 + 16 * j;
#pragma unroll
        for (int c = 0; c < kSplitChunks; ++c) {
            const int64_t chunk = k0 / kSkinnyChunk + c;
            if (TILED) {
                const char* pj = bbase + ((brow / 16) * chunk_count + chunk) * kTileBytes + lane * 16;
#pragma unroll
                for (int s = 0; s < BQ; ++s) bq[c][j][s] = *reinterpret_cast<const uint4*>(pj + 1024 * s);
            } else {
                const int64_t belem = (BDT == SFG_I8) ? 1 : 2;
                const char* pj = bbase + ((brow + lr) * p.ldb + chunk * kSkinnyChunk + lg * kLaneK) * belem;
#pragma unroll
                for (int s = 0; s < BQ; ++s)
                    bq[c][j][s] = *reinterpret_cast<const uint4*>(pj + (BDT == SFG_I8 ? 16 * s : 2 * kStepK * s));
            }
        }
    }
    // 3. activations -> LDS
#pragma unroll
    for (int i = 0; i < kStageVecs; ++i) {
        const int q = tid + 256 * i;
        const int row = q / kVecsPerRow, v = q % kVecsPerRow;
        *reinterpret_cast<uint4*>(&sa[row * kSplitLdA + 8 * v]) = row < p.m ? av[i] : make_uint4(0, 0, 0, 0);
    }
    // LDS stores done, weight loads still in flight across the barrier
    wait_lds();
    barrier_no_fence();

    // 4. MFMAs: A fragments from LDS in the k order of the weight fragments
    floatx4 acc[4][kSplitTiles];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kSplitTiles; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < kSplitChunks; ++c) {
        bf16x8 bf[kSplitTiles][4];
#pragma unroll
        for (int j = 0; j < kSplitTiles; ++j) {
            if (BDT == SFG_I8) {
                bf[j][0] = as_bf16x8(i8x8_to_bf16x8(bq[c][j][0].x, bq[c][j][0].y));
                bf[j][1] = as_bf16x8(i8x8_to_bf16x8(bq[c][j][0].z, bq[c][j][0].w));
                bf[j][2] = as_bf16x8(i8x8_to_bf16x8(bq[c][j][1].x, bq[c][j][1].y));
                bf[j][3] = as_bf16x8(i8x8_to_bf16x8(bq[c][j][1].z, bq[c][j][1].w));
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) bf[j][s] = as_bf16x8(bq[c][j][s]);
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kk = c * kSkinnyChunk + lg * kLaneK + s * kStepK;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(&sa[(16 * i + lr) * kSplitLdA + kk]));
#pragma unroll
                for (int j = 0; j < kSplitTiles; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bf[j][s], acc[i][j], 0, 0, 0);
            }
        }
    }
    // 5. partial sums: lane holds column lr, rows 4 lg + r of each 16-row tile
    float* part = p.part + static_cast<int64_t>(blockIdx.y) * p.m * p.nb;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = 16 * i + 4 * lg + r;
            if (row >= p.m) continue;
#pragma unroll
            for (int j = 0; j < kSplitTiles; ++j) part[row * p.nb + col0 + 16 * j + lr] = acc[i][j][r];
        }
}

struct SplitReduceArgs {
    const float* part; int slices;
    const float* scales;
    void* c; int c_dtype; int64_t ldc;
    const float* residual; int64_t ldr;
    int64_t m, n, nb;  // n output columns; nb = B rows (2 n for GLU)
};

template <int EPI>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(SplitReduceArgs p) {
    // four consecutive output columns per thread (n is a multiple of 64); the
    // slices' loads are all issued before the ordered sum
    const int64_t idx = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (idx >= p.m * p.n) return;
    const int64_t row = idx / p.n, col = idx % p.n;
    const int64_t stride = p.m * p.nb;
    const float* pr = p.part + row * p.nb + col;
    constexpr int kBatch = 8;  // slices loaded together, then added in order
    constexpr bool kGlu = EpiTraits<EPI>::glu;
    // The epilogue's scales and residual values are read before any store:
    // the output may alias them for all the compiler knows, so loads placed
    // after a store would each wait a full memory round trip.
    float sg[4], su[4], rv[4];
    if (p.scales) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sg[e] = p.scales[col + e];
            if constexpr (kGlu) su[e] = p.scales[p.n + col + e];
        }
    }
    if constexpr (EPI == SFG_EPI_RESIDUAL) {
#pragma unroll
        for (int e = 0; e < 4; ++e) rv[e] = p.residual[row * p.ldr + col + e];
    }
    float gv[4] = {0.f, 0.f, 0.f, 0.f}, uv[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < p.slices; s0 += kBatch) {
        float4 g[kBatch], u[kGlu ? kBatch : 1];
#pragma unroll
        for (int s = 0; s < kBatch; ++s) {
            if (s0 + s < p.slices) {
                g[s] = *reinterpret_cast<const float4*>(pr + (s0 + s) * stride);
                if constexpr (kGlu) u[s] = *reinterpret_cast<const float4*>(pr + (s0 + s) * stride + p.n);
            }
        }
#pragma unroll
        for (int s = 0; s < kBatch; ++s) {
            if (s0 + s < p.slices) {
                gv[0] += g[s].x; gv[1] += g[s].y; gv[2] += g[s].z; gv[3] += g[s].w;
                if constexpr (kGlu) { uv[0] += u[s].x; uv[1] += u[s].y; uv[2] += u[s].z; uv[3] += u[s].w; }
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int64_t cc = col + e;
        if (kGlu) {
            float gg = gv[e], uu = uv[e];
            if (p.scales) {
                gg *= sg[e];
                uu *= su[e];
            }
            store_out(p.c, p.c_dtype, row * p.ldc + cc, glu_combine(EPI, gg, uu));
        } else {
            float v = gv[e];
            if (p.scales) v *= sg[e];
            if (EPI == SFG_EPI_RESIDUAL) v += rv[e];
            store_out(p.c, p.c_dtype, row * p.ldc + cc, v);
        }
    }
}

// ===========================================================================
// Large-M MFMA GEMM: 128x128 output tile, BK = 32, 4 waves in a 2x2 grid, each
// wave 64x64 = 2x2 tiles of v_mfma_f32_32x32x16_bf16.
// LDS holds A[128][32] and B[128][32] bf16 with rows padded to 80 B so that the
// 16-byte fragment reads of 32 consecutive rows spread over the banks.
// ===========================================================================
struct TiledArgs {
    const uint16_t* a; int64_t lda; const int32_t* a_rows; int64_t a_rows_limit;
    const void* b; int64_t ldb; const float* scales;
    int64_t b_group_stride, s_group_stride;
    void* c; int c_dtype; int64_t ldc;
    const float* residual; int64_t ldr;
    int64_t m, n, k;
    const int32_t* offsets;   // grouped: tiles per group = ceil(rows_g / 128)
    int groups;
    QkvRopeOut qkv;           // kEpiQkvRope only
    int xcds;                 // XCDs the dispatcher deals workgroups over
};

constexpr int kTM = 128, kTN = 128, kTK = 32;
constexpr int kLdsRow = 40;  // bf16 elements per padded LDS row (32 + 8)

template <int BDT, int EPI>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(TiledArgs p) {
    constexpr bool kGlu = EpiTraits<EPI>::glu;
    __shared__ __attribute__((aligned(16))) uint16_t sA[kTM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint16_t sB[kTN * kLdsRow];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // Map blockIdx.y to (group, row tile).
    int g = 0;
    int64_t rb = 0, re = p.m;
    int64_t mtile = blockIdx.y;
    if (p.offsets) {
        int64_t t = blockIdx.y;
        g = -1;
        auto bound = [&](int e) {
            return min(max(static_cast<int64_t>(p.offsets[e]), int64_t(0)), p.m);
        };
        for (int e = 0; e < p.groups; ++e) {
            const int64_t lo = bound(e);
            const int64_t rows = max(bound(e + 1) - lo, int64_t(0));
            const int64_t tiles = (rows + kTM - 1) / kTM;
            if (t < tiles) { g = e; break; }
            t -= tiles;
        }
        if (g < 0) return;
        rb = bound(g);
        re = max(bound(g + 1), rb);
        mtile = t;
    }
    const int64_t row0 = rb + mtile * kTM;
    if (row0 >= re) return;

    // Output columns of this tile.  GLU: 64 gate + 64 up B rows -> 64 outputs.
    const int64_t ncol0 = static_cast<int64_t>(blockIdx.x) * (kGlu ? kTN / 2 : kTN);
    const int64_t bgroup = static_cast<int64_t>(g) * p.b_group_stride;
    const float* scales = p.scales ? p.scales + static_cast<int64_t>(g) * p.s_group_stride : nullptr;

    // Global -> LDS loaders: each thread moves 16 B of A and 16 B of B per slab
    // (128 rows x 32 k x 2 B = 8 KB = 256 threads x 2 x 16 B -> two per thread).
    // Output columns at or past n (a ragged last tile) read B row 0 instead;
    // their results are never stored.
    int64_t a_src[2];
    bool a_ok[2];
    int64_t b_src[2];
    int ld_row[2], ld_col[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int idx = tid + h * 256;     // 0..511
        ld_row[h] = idx >> 2;              // 0..127
        ld_col[h] = (idx & 3) * 8;         // 0,8,16,24
        const int64_t r = row0 + ld_row[h];
        a_ok[h] = r < re;
        int64_t src = a_ok[h] ? (p.a_rows ? p.a_rows[r] : r) : 0;
        if (src < 0 || src >= p.a_rows_limit) { a_ok[h] = false; src = 0; }
        a_src[h] = src * p.lda + ld_col[h];
        int64_t brow;
        if (kGlu) {
            const int local = ld_row[h];
            const int64_t col = ncol0 + (local & 63);
            brow = col < p.n ? ((local < 64) ? col : p.n + col) : 0;
        } else {
            const int64_t col = ncol0 + ld_row[h];
            brow = col < p.n ? col : 0;
        }
        b_src[h] = bgroup + brow * p.ldb + ld_col[h];
    }
    const char* bbytes = static_cast<const char*>(p.b);

    auto fetch = [&](int64_t k0, uint4 (&ra)[2], uint4 (&rbv)[2]) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            ra[h] = a_ok[h] ? *reinterpret_cast<const uint4*>(p.a + a_src[h] + k0) : make_uint4(0, 0, 0, 0);
            if (BDT == SFG_I8) {
                const uint2 q = *reinterpret_cast<const uint2*>(bbytes + b_src[h] + k0);
                rbv[h] = i8x8_to_bf16x8(q.x, q.y);
            } else {
                rbv[h] = *reinterpret_cast<const uint4*>(bbytes + (b_src[h] + k0) * 2);
            }
        }
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    uint4 ra[2], rbv[2];
    fetch(0, ra, rbv);
    const int64_t ksteps = p.k / kTK;
    for (int64_t kt = 0; kt < ksteps; ++kt) {
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            *reinterpret_cast<uint4*>(&sA[ld_row[h] * kLdsRow + ld_col[h]]) = ra[h];
            *reinterpret_cast<uint4*>(&sB[ld_row[h] * kLdsRow + ld_col[h]]) = rbv[h];
        }
        __syncthreads();
        if (kt + 1 < ksteps) fetch((kt + 1) * kTK, ra, rbv);
        // Two MFMA k-steps of 16 per slab.  Operand lane layout (32x32x16):
        // lane l supplies row/col (l & 31), k = (l >> 5) * 8 + [0, 8).
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            bf16x8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = wm * 64 + i * 32 + (lane & 31);
                af[i] = as_bf16x8(*reinterpret_cast<const uint4*>(
                    &sA[r * kLdsRow + kk * 16 + (lane >> 5) * 8]));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                int r;
                if (kGlu) r = (j == 0 ? 0 : 64) + wn * 32 + (lane & 31);
                else r = wn * 64 + j * 32 + (lane & 31);
                bf[j] = as_bf16x8(*reinterpret_cast<const uint4*>(
                    &sB[r * kLdsRow + kk * 16 + (lane >> 5) * 8]));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }

    // Epilogue.  32x32 D layout: lane l holds column (l & 31) and rows
    // 8 * (r / 4) + 4 * (l >> 5) + (r % 4) for r = 0..15.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int lrow = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int64_t row = row0 + lrow;
            if (row >= re) continue;
            if (kGlu) {
                const int64_t col = ncol0 + wn * 32 + (lane & 31);
                if (col >= p.n) continue;
                float gv = acc[i][0][r], uv = acc[i][1][r];
                if (scales) {
                    gv *= scales[col];
                    uv *= scales[p.n + col];
                }
                store_out(p.c, p.c_dtype, row * p.ldc + col, glu_combine(EPI, gv, uv));
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int64_t col = ncol0 + wn * 64 + j * 32 + (lane & 31);
                    if (col >= p.n) continue;
                    float v = acc[i][j][r];
                    if (scales) v *= scales[col];
                    if (EPI == SFG_EPI_RESIDUAL) v += p.residual[row * p.ldr + col];
                    store_out(p.c, p.c_dtype, row * p.ldc + col, v);
                }
            }
        }
    }
}

// ===========================================================================
// Large-M MFMA GEMM, second generation: 256x128 output tile per workgroup (for
// GLU epilogues 256 rows x 64 outputs, i.e. 64 gate + 64 up B rows), BK = 64.
// Four waves each own 64 rows x 128 B-columns = 2 x 4 tiles of
// v_mfma_f32_32x32x16_bf16 (128 fp32 accumulators per lane).  The k-slabs are
// double-buffered in LDS (rows padded to 144 B), the next slab is fetched into
// registers while the current one feeds the MFMAs, and there is one barrier
// per slab.  Dense problems map workgroups XCD-aware: consecutive workgroup
// ids are spread over the 8 XCDs by the dispatcher, so each XCD is handed a
// contiguous run of tiles in grouped (8 M-tiles) order, which shares A and B
// tiles inside one L2.
// ===========================================================================
constexpr int kGM = 256, kGN = 128, kGK = 64;
constexpr int kGRow = kGK + 8;  // padded LDS row, bf16 elements

template <int BDT, int EPI>
__global__ __launch_bounds__(256) void gemm_mfma256_kernel(TiledArgs p, int tiles_m, int tiles_n) {
    constexpr bool kGlu = EpiTraits<EPI>::glu;
    __shared__ __attribute__((aligned(16))) uint16_t sA[2][kGM * kGRow];
    __shared__ __attribute__((aligned(16))) uint16_t sB[2][kGN * kGRow];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    int g = 0;
    int64_t rb = 0, re = p.m;
    int64_t tm, tn;
    if (p.offsets) {
        tn = blockIdx.x;
        int64_t t = blockIdx.y;
        auto bound = [&](int e) {
            return min(max(static_cast<int64_t>(p.offsets[e]), int64_t(0)), p.m);
        };
        g = -1;
        for (int e = 0; e < p.groups; ++e) {
            const int64_t rows = max(bound(e + 1) - bound(e), int64_t(0));
            const int64_t tiles = (rows + kGM - 1) / kGM;
            if (t < tiles) { g = e; break; }
            t -= tiles;
        }
        if (g < 0) return;
        rb = bound(g);
        re = max(bound(g + 1), rb);
        tm = t;
    } else {
        const int64_t total = static_cast<int64_t>(tiles_m) * tiles_n;
        const int64_t i = blockIdx.x;
        const int64_t x = p.xcds;
        const int64_t full = total - total % x;
        int64_t L = i;
        if (i < full) L = (i % x) * (full / x) + i / x;
        constexpr int64_t kGroupM = 8;
        const int64_t group = L / (kGroupM * tiles_n);
        const int64_t first_m = group * kGroupM;
        const int64_t gsize = min(static_cast<int64_t>(tiles_m) - first_m, kGroupM);
        const int64_t in_group = L % (kGroupM * tiles_n);
        tm = first_m + in_group % gsize;
        tn = in_group / gsize;
    }
    const int64_t row0 = rb + tm * kGM;
    if (row0 >= re) return;
    const int64_t ncol0 = tn * (kGlu ? kGN / 2 : kGN);
    const int64_t bgroup = static_cast<int64_t>(g) * p.b_group_stride;
    const float* scales = p.scales ? p.scales + static_cast<int64_t>(g) * p.s_group_stride : nullptr;

    // Global -> register staging: A 256 x 64 = 8 chunks of 16 B per thread,
    // B 128 x 64 = 4 chunks.  Chunk (row, kc): row = (tid >> 3) + 32 i, kc = 8 (tid & 7).
    const int kc = (tid & 7) * 8;
    const uint16_t* a_src[8];
    bool a_ok[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t r = row0 + (tid >> 3) + 32 * i;
        a_ok[i] = r < re;
        int64_t src = a_ok[i] ? (p.a_rows ? p.a_rows[r] : r) : 0;
        if (src < 0 || src >= p.a_rows_limit) { a_ok[i] = false; src = 0; }
        a_src[i] = p.a + src * p.lda + kc;
    }
    const char* bbytes = static_cast<const char*>(p.b);
    int64_t b_src[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int local = (tid >> 3) + 32 * i;
        int64_t brow;
        if (kGlu) brow = local < 64 ? ncol0 + local : p.n + ncol0 + local - 64;
        else brow = ncol0 + local;
        b_src[i] = bgroup + brow * p.ldb + kc;  // elements
    }
    uint4 ra[8], rbv[4];
    auto fetch = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            ra[i] = a_ok[i] ? *reinterpret_cast<const uint4*>(a_src[i] + k0) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (BDT == SFG_I8) {
                const uint2 q = *reinterpret_cast<const uint2*>(bbytes + b_src[i] + k0);
                rbv[i] = i8x8_to_bf16x8(q.x, q.y);
            } else {
                rbv[i] = *reinterpret_cast<const uint4*>(bbytes + (b_src[i] + k0) * 2);
            }
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<uint4*>(&sA[buf][((tid >> 3) + 32 * i) * kGRow + kc]) = ra[i];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<uint4*>(&sB[buf][((tid >> 3) + 32 * i) * kGRow + kc]) = rbv[i];
    };

    floatx16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int64_t slabs = p.k / kGK;
    fetch(0);
    stash(0);
    __syncthreads();
    const int l32 = lane & 31, lh = (lane >> 5) * 8;
    for (int64_t kt = 0; kt < slabs; ++kt) {
        const int cur = static_cast<int>(kt & 1);
        if (kt + 1 < slabs) fetch((kt + 1) * kGK);
        const uint16_t* A = sA[cur];
        const uint16_t* B = sB[cur];
#pragma unroll
        for (int kk = 0; kk < kGK / 16; ++kk) {
            bf16x8 af[2], bf[4];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = as_bf16x8(*reinterpret_cast<const uint4*>(
                    &A[(wave * 64 + i * 32 + l32) * kGRow + kk * 16 + lh]));
#pragma unroll
            for (int j = 0; j < 4; ++j)
                bf[j] = as_bf16x8(*reinterpret_cast<const uint4*>(
                    &B[(j * 32 + l32) * kGRow + kk * 16 + lh]));
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < slabs) stash(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: 32x32 D layout, lane holds column (lane & 31) and rows
    // 8 (r / 4) + 4 (lane >> 5) + (r % 4).
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = row0 + wave * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (row >= re) continue;
            if (kGlu) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int64_t col = ncol0 + j * 32 + l32;
                    float gv = acc[i][j][r], uv = acc[i][j + 2][r];
                    if (scales) {
                        gv *= scales[col];
                        uv *= scales[p.n + col];
                    }
                    store_out(p.c, p.c_dtype, row * p.ldc + col, glu_combine(EPI, gv, uv));
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t col = ncol0 + j * 32 + l32;
                    float v = acc[i][j][r];
                    if (scales) v *= scales[col];
                    if (EPI == SFG_EPI_RESIDUAL) v += p.residual[row * p.ldr + col];
                    store_out(p.c, p.c_dtype, row * p.ldc + col, v);
                }
            }
        }
    }
}

// ===========================================================================
// QKV epilogue for the bf16 prefill (split_qkv + apply_rope,
// decoder_compiler.cpp:96-148, plus the transposed V the flash prefill reads):
// the [rows][H + 2 Hkv 128] product is never stored.  Column c of the
// accumulator lives in lane c % 32; RoPE pairs (2i, 2i+1) are neighbouring
// lanes of one row, so one lane exchange gives each lane its partner, and the
// rotation is split_rope_kernel's expression (same table, same float ops).
// Every 32-column block lies inside one head, so the Q / K / V choice is
// uniform per block.  A lane's four consecutive rows (r % 4) are four
// consecutive tokens of one sequence (S % 4 == 0, checked on the host), so
// V^T takes one 8-byte store per lane and block.
// ===========================================================================
template <int WM, int WN>
__device__ __forceinline__ void qkv_rope_epilogue(const QkvRopeOut& o, const floatx16 (&acc)[WM][WN],
                                                  int64_t wave_row0, int64_t wave_col0, int64_t re,
                                                  int64_t n, int l32, int khalf) {
    const int64_t H = static_cast<int64_t>(o.q_heads) * 128;
    const int64_t kvd = static_cast<int64_t>(o.kv_heads) * 128;
    const int seq = static_cast<int>(o.seq);
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        // One 32-row block: positions and (cos, sin) of all its rows and this
        // lane's columns are fetched first, so the block waits for the table
        // once instead of once per element.
        int bq[4], sq[4];
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
            const int rr = static_cast<int>(wave_row0 + i * 32 + 8 * rq + 4 * khalf);
            bq[rq] = rr / seq;
            sq[rq] = rr - bq[rq] * seq;
        }
        float2 cs[WN][4][4];
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const int64_t col = wave_col0 + j * 32 + l32;
            const bool rot = col < H + kvd;  // uniform over the 32-column block
            const int pr = static_cast<int>(col & 127) >> 1;
#pragma unroll
            for (int rq = 0; rq < 4; ++rq)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    cs[j][rq][e] = rot ? o.rope[static_cast<int64_t>(sq[rq] + e) * 64 + pr] : make_float2(1.f, 0.f);
        }
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
            const int64_t row = wave_row0 + i * 32 + 8 * rq + 4 * khalf;  // rows row .. row + 3
            const int b = bq[rq], s0 = sq[rq];
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int64_t col = wave_col0 + j * 32 + l32;
                float v[4], pv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = acc[i][j][4 * rq + e];
                    pv[e] = __shfl_xor(v[e], 1, 64);
                }
                if (col >= n || row >= re) continue;
                const int d = static_cast<int>(col & 127);
                if (col < H + kvd) {
                    uint16_t* dst = col < H
                        ? o.q + ((static_cast<int64_t>(b) * o.q_heads + (col >> 7)) * seq + s0) * 128 + d
                        : o.k + ((static_cast<int64_t>(b) * o.kv_heads + ((col - H) >> 7)) * seq + s0) * 128 + d;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float2 c = cs[j][rq][e];
                        // (even, odd) -> (even c - odd s, odd c + even s), the same
                        // fused operations as qkv_rope_epilogue_staged
                        const float r0 = (d & 1) ? fmaf(v[e], c.x, pv[e] * c.y) : fmaf(v[e], c.x, -(pv[e] * c.y));
                        dst[e * 128] = f32_to_bf16(r0);
                    }
                } else {
                    const int64_t hv = (col - H - kvd) >> 7;
                    uint2 pk;
                    pk.x = pack_bf16x2(v[0], v[1]);
                    pk.y = pack_bf16x2(v[2], v[3]);
                    *reinterpret_cast<uint2*>(o.vt + ((static_cast<int64_t>(b) * o.kv_heads + hv) * 128 + d) * o.ld_vt + s0) = pk;
                }
            }
        }
    }
}

// The same epilogue for a wave's block of a four-wave tile (128 x 128 of a
// 256 x 256 tile, or 64 x 64 of a 128 x 128 one), through the wave's own LDS
// stage array: for each 32-row block the accumulators go to LDS as fp32
// [32][kCols] (column c of row r at c ^ ((r & 4) << 3), so the two row halves
// of a write use different banks), then every lane reads 8 consecutive
// columns of one row, rotates its 4 pairs with a 32-byte read of the
// (cos, sin) table (issued one row block ahead) and writes 16 bytes of Q or K.
// A V^T block is staged transposed and leaves as 16-byte runs of positions; a
// block past the last column, or V^T when the sequence length is not a
// multiple of 8, takes the per-lane path.
template <int WM, int WN>
__device__ __forceinline__ void qkv_rope_epilogue_staged(const QkvRopeOut& o, const floatx16 (&acc)[WM][WN],
                                                         int64_t wave_row0, int64_t wave_col0, int64_t re,
                                                         int64_t n, int lane, float* stage) {
    static_assert((WM == 4 && WN == 4) || (WM == 2 && WN == 2), "128 x 128 or 64 x 64 per wave");
    constexpr int kCols = 32 * WN;          // columns of the wave block (within one head)
    constexpr int kPos = 32 * WM;           // rows (positions) of the wave block
    const int l32 = lane & 31, khalf = lane >> 5;
    const int64_t H = static_cast<int64_t>(o.q_heads) * 128;
    const int64_t kvd = static_cast<int64_t>(o.kv_heads) * 128;
    const int64_t seq = o.seq;
    if (wave_col0 + kCols > n || (wave_col0 >= H + kvd && seq % 8 != 0)) {
        qkv_rope_epilogue<WM, WN>(o, acc, wave_row0, wave_col0, re, n, l32, khalf);
        return;
    }
    const int col_in_head = static_cast<int>(wave_col0 & 127);  // 0, or 64 for 64-column blocks
    if (wave_col0 >= H + kvd) {
        // V^T block: bf16 [kCols d][kPos s] in LDS; 8-byte granule g of row d
        // sits at g ^ x(d), which spreads the 32 rows of a write over distinct
        // bank pairs (rows are 256 B apart for kPos 128, 128 B for 64).
        // Then 16-byte runs of 8 positions of one d row go out whole.
        constexpr int kGran = kPos / 4;
        auto swz = [](int d) { return kGran == 32 ? (d & 31) : ((d >> 1) & (kGran - 1)); };
        uint16_t* const st = reinterpret_cast<uint16_t*>(stage);
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int rq = 0; rq < 4; ++rq) {
                    const int d = j * 32 + l32;
                    const int g = i * 8 + 2 * rq + khalf;  // positions 4 g .. 4 g + 3
                    uint2 pk;
                    pk.x = cvt_pk_bf16(acc[i][j][4 * rq + 0], acc[i][j][4 * rq + 1]);
                    pk.y = cvt_pk_bf16(acc[i][j][4 * rq + 2], acc[i][j][4 * rq + 3]);
                    *reinterpret_cast<uint2*>(st + d * kPos + (g ^ swz(d)) * 4) = pk;
                }
        constexpr int kRunLanes = kPos / 8;         // lanes per d row (8 positions each)
        constexpr int kRowsPer = 64 / kRunLanes;    // d rows per instruction
        const int64_t hv = (wave_col0 - H - kvd) >> 7;
        const int c = lane % kRunLanes;             // positions 8 c .. 8 c + 7 of a d row
        const int64_t grow = wave_row0 + 8 * c;     // first of the 8 rows
        const int64_t b = static_cast<uint32_t>(grow) / static_cast<uint32_t>(seq);
        const int64_t sp = grow - b * seq;
        uint16_t* const dst0 = o.vt + ((b * o.kv_heads + hv) * 128 + col_in_head) * o.ld_vt + sp;
#pragma unroll
        for (int t = 0; t < kCols / kRowsPer; ++t) {
            const int d = kRowsPer * t + lane / kRunLanes;
            const int x = swz(d);
            uint4 v = *reinterpret_cast<const uint4*>(st + d * kPos + ((2 * c) ^ (x & ~1)) * 4);
            if (x & 1) v = make_uint4(v.z, v.w, v.x, v.y);  // the two granules of the run swapped
            uint16_t* const dst = dst0 + d * o.ld_vt;
            if (grow + 8 <= re && sp + 8 <= seq) {
                *reinterpret_cast<uint4*>(dst) = v;
            } else {
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int64_t r = grow + e;
                    if (r >= re) break;
                    const int64_t be = r / seq, se = r - be * seq;
                    o.vt[((be * o.kv_heads + hv) * 128 + col_in_head + d) * o.ld_vt + se] =
                        static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
                }
            }
        }
        return;
    }
    const bool isq = wave_col0 < H;
    uint16_t* const base = isq ? o.q : o.k;
    const int64_t heads = isq ? o.q_heads : o.kv_heads;
    const int64_t head = isq ? (wave_col0 >> 7) : ((wave_col0 - H) >> 7);
    constexpr int kChunkLanes = kCols / 8;        // lanes per row when reading back
    constexpr int kRowsPer = 64 / kChunkLanes;    // rows per read-back step
    constexpr int kSteps = 32 / kRowsPer;         // steps per 32-row block
    const int c8 = lane % kChunkLanes;            // this lane's 8-column chunk
    const int lrow = lane / kChunkLanes;
    // (sequence, position) of this lane's first row in block i.  Its rows are
    // kRowsPer t + lrow, so later ones advance the position by kRowsPer,
    // wrapping into the next sequence: one division per block (rows and the
    // sequence length fit 32 bits on this path) instead of one per row.
    const uint32_t useq = static_cast<uint32_t>(seq);
    auto block_pos = [&](int i, uint32_t& b, uint32_t& sp) {
        const uint32_t g = static_cast<uint32_t>(wave_row0 + i * 32 + lrow);
        b = g / useq;
        sp = g - b * useq;
    };
    auto next_pos = [&](uint32_t& b, uint32_t& sp) {
        sp += kRowsPer;
        if (sp >= useq) {  // a sequence boundary (several when seq < kRowsPer)
            const uint32_t q = sp / useq;
            b += q;
            sp -= q * useq;
        }
    };
    // (cos, sin) of this lane's 4 pairs for its rows of block i: all table
    // reads of a block are issued one block ahead, so the block never waits
    // for the table.  (Rows past the end read a valid row, unused.)
    const int pair0 = col_in_head / 2 + c8 * 4;
    auto table = [&](int i, float4 (&cs)[kSteps][2]) {
        uint32_t bt, sp;
        block_pos(i, bt, sp);
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            if (t) next_pos(bt, sp);
            const float4* src = reinterpret_cast<const float4*>(o.rope + static_cast<int64_t>(sp) * 64 + pair0);
            cs[t][0] = src[0];
            cs[t][1] = src[1];
        }
    };
    float4 cs[2][kSteps][2];
    table(0, cs[0]);
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        if (i + 1 < WM) table(i + 1, cs[(i + 1) & 1]);
        // LDS accesses of one wave complete in order: the reads below see
        // these writes, and the next block's writes follow these reads.
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 8 * (r >> 2) + 4 * khalf + (r & 3);
                stage[row * kCols + ((j * 32 + l32) ^ ((row & 4) << 3))] = acc[i][j][r];
            }
        uint32_t b, sp;
        block_pos(i, b, sp);
#pragma unroll
        for (int t = 0; t < kSteps; ++t) {
            if (t) next_pos(b, sp);
            const int row = kRowsPer * t + lrow;
            const float* src = stage + row * kCols + ((c8 * 8) ^ ((row & 4) << 3));
            const float4 v0 = *reinterpret_cast<const float4*>(src);
            const float4 v1 = *reinterpret_cast<const float4*>(src + 4);
            const int64_t grow = wave_row0 + i * 32 + row;
            if (grow >= re) continue;
            const float4 cs0 = cs[i & 1][t][0], cs1 = cs[i & 1][t][1];  // this lane's 4 pairs
            // hardware RNE pair conversion: the same bits as pack_bf16x2 for finite values
            auto rot = [](float e, float od, float c, float sn) {
                return cvt_pk_bf16(fmaf(e, c, -(od * sn)), fmaf(od, c, e * sn));
            };
            uint4 pk;
            pk.x = rot(v0.x, v0.y, cs0.x, cs0.y);
            pk.y = rot(v0.z, v0.w, cs0.z, cs0.w);
            pk.z = rot(v1.x, v1.y, cs1.x, cs1.y);
            pk.w = rot(v1.z, v1.w, cs1.z, cs1.w);
            *reinterpret_cast<uint4*>(base + ((static_cast<int64_t>(b) * heads + head) * seq + sp) * 128 +
                                      col_in_head + c8 * 8) = pk;
        }
    }
}

// GLU store epilogue of a wave's 128 x 64 output block in the four-wave
// 256 x 256 tile (bf16 out), through a 16 KB LDS region of its own: the
// silu-combined values go to LDS as bf16 [128 rows][64 columns] (column c of
// row r at c ^ ((r & 4) << 3), so the two row halves of a write hit different
// banks), then every lane stores 16-byte row chunks, instead of one 2-byte
// element per lane per store instruction.  The arithmetic is the generic
// epilogue's, value for value.
template <int EPI>
__device__ __forceinline__ void glu_epilogue_staged(const TiledArgs& p, const floatx16 (&acc)[4][4],
                                                    int64_t wrow0, int64_t wcol0, int64_t re,
                                                    const float* scales, int lane, uint16_t* stage) {
    const int l32 = lane & 31, khalf = lane >> 5;
    // wcol0: the first of this wave's 64 output columns
    float sc_lo[2], sc_hi[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int64_t cc = min(wcol0 + j * 32 + l32, p.n - 1);
        sc_lo[j] = scales ? scales[cc] : 1.f;
        sc_hi[j] = scales ? scales[p.n + cc] : 1.f;
    }
    // Two rows at a time through the hardware RNE converter (the same bits as
    // f32_to_bf16 for finite values); unscaled weights skip the multiplies.
    auto combine_rows = [&](auto scaled_c) __attribute__((always_inline)) {
        constexpr bool kScaled = decltype(scaled_c)::value;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    float v[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const float g = kScaled ? acc[i][2 * j][r + e] * sc_lo[j] : acc[i][2 * j][r + e];
                        const float u = kScaled ? acc[i][2 * j + 1][r + e] * sc_hi[j] : acc[i][2 * j + 1][r + e];
                        v[e] = glu_combine(EPI, g, u);
                    }
                    const uint32_t pk = cvt_pk_bf16(v[0], v[1]);
                    const int row = i * 32 + 8 * (r >> 2) + 4 * khalf + (r & 3);  // rows row, row + 1
                    const int col = j * 32 + l32;
                    stage[row * 64 + (col ^ ((row & 4) << 3))] = static_cast<uint16_t>(pk);
                    stage[(row + 1) * 64 + (col ^ (((row + 1) & 4) << 3))] = static_cast<uint16_t>(pk >> 16);
                }
    };
    if (scales) combine_rows(std::true_type{});
    else combine_rows(std::false_type{});
    // a wave's LDS accesses complete in order: the reads see the writes
    uint16_t* const out = static_cast<uint16_t*>(p.c);
    const int c8 = lane & 7;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        const int row = t * 8 + (lane >> 3);
        const uint4 v = *reinterpret_cast<const uint4*>(stage + row * 64 + ((c8 * 8) ^ ((row & 4) << 3)));
        const int64_t grow = wrow0 + row, col = wcol0 + c8 * 8;
        if (grow >= re) continue;
        uint16_t* const dst = out + grow * p.ldc + col;
        if (col + 8 <= p.n) {
            *reinterpret_cast<uint4*>(dst) = v;
        } else {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (col + e < p.n) dst[e] = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
        }
    }
}

// ===========================================================================
// Large-M MFMA GEMM, third generation (bf16 operands): BM x BN output tile per
// workgroup, four waves in a 2 x 2 grid, each owning a (BM/2) x (BN/2) block of
// v_mfma_f32_32x32x16_bf16 tiles (accumulators in the AccVGPRs).
// K advances in slabs of 32 through a ring of LDS stages (four, or three for
// the two-workgroups-per-CU tiles): the operand slabs go from global memory
// straight into LDS (global_load_lds_dwordx4, one wave instruction fills one
// contiguous 1 KB block = 16 rows x 32 k of bf16), and the next slabs are in
// flight while one is multiplied (one __shared__ array per stage: the A slab,
// then the B slab).  Before slab k is
// read each wave waits only for its own loads of slab k (vmcnt = the loads of
// the slabs issued after it), then a barrier makes every wave's loads visible
// and retires the stage the next issue overwrites.
// Rows are 64 B = 4 chunks of 16 B; chunk c of row r sits in slot
// c ^ ((r >> 2) & 3), so the fragment reads of 16 consecutive rows (one LDS
// pass of 16 lanes over 64 banks) touch 16 distinct 16-byte bank groups.  The
// loading lane picks the chunk it fetches so its fixed destination slot holds
// the swizzled one.  Each stage lives in its own __shared__ array, so the
// compiler can tell the in-flight loads from the stage being read.
// For GLU epilogues the B tile interleaves 32-row blocks of gate and up rows
// (block 2j: gate columns j*32.., block 2j+1: the same up columns), so every
// lane holds matching gate and up accumulators.
// ===========================================================================
constexpr int kRK = 32;

// Stages and workgroups per CU by tile: 256 x 256 holds 256 accumulator
// registers per lane (one workgroup per CU, four stages = 128 KB of LDS);
// smaller tiles leave room for two workgroups per CU, so one's barriers and
// epilogue overlap the other's MFMAs (256 x 128: three stages = 72 KB each).
// With eight waves (2 x 4) a 256 x 256 tile keeps 128 accumulator registers
// per lane and two waves per SIMD, so one wave's LDS waits overlap the other's
// MFMAs.
// Scheduling groups for one interleaved half slab: NM MFMAs; the NR LDS reads
// of the next half go one after each of the first MFMAs (so the last has most
// of the half to land before its MFMA needs it), and the NV VMEM loads are
// spread over the MFMAs after them.
template <int NM, int NR, int NV, int I = 0>
__device__ __forceinline__ void interleave_groups() {
    if constexpr (I < NM) {
        constexpr int kRest = NM - (NR < NM ? NR : NM);  // MFMAs after the reads
        constexpr int kJ = I - (NM - kRest);              // index among them
        constexpr int kLoadsHere = (NV == 0 || kJ < 0) ? 0
            : (kRest == 0 ? (I == NM - 1 ? NV : 0) : (kJ + 1) * NV / kRest - kJ * NV / kRest);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if constexpr (I < NR) __builtin_amdgcn_sched_group_barrier(0x100, I == NM - 1 ? NR - I : 1, 0);  // DS read
        if constexpr (kLoadsHere > 0) __builtin_amdgcn_sched_group_barrier(0x020, kLoadsHere, 0);  // VMEM read
        interleave_groups<NM, NR, NV, I + 1>();
    }
}

// Scheduling groups for a run of NM MFMAs that also reads fragments and
// issues loads: one LDS fragment read after each of the first NR MFMAs, and NV
// VMEM instructions (LDS DMA) spread evenly over all NM, so the four waves of
// a CU never queue a burst of LDS reads or of DMA requests.
template <int NM, int NR, int NV, int I = 0>
__device__ __forceinline__ void spread_reads_loads() {
    if constexpr (I < NM) {
        constexpr int loads = (I + 1) * NV / NM - I * NV / NM;
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                          // MFMA
        if constexpr (I < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);       // DS read
        if constexpr (loads > 0) __builtin_amdgcn_sched_group_barrier(0x020, loads, 0);  // VMEM
        spread_reads_loads<NM, NR, NV, I + 1>();
    }
}

template <int BM, int BN, int NW>
struct DmaShapeTraits {
    static constexpr bool big = BM * BN > 256 * 128;
    static constexpr int stages = (big || BM * BN <= 128 * 128) ? 4 : 3;
    static constexpr int occupancy = (big && NW == 4) ? 1 : 2;
    // The four-wave 256 x 256 tile has registers for two full fragment sets
    // (its accumulators live in AGPRs): it reads a whole slab ahead.
    static constexpr bool slab_ahead = big && NW == 4;
    static constexpr int dma_bytes = 16;  // per lane per LDS DMA instruction (dwordx4)
};

// Tile of this workgroup in a direct-to-LDS launch.  Grouped (p.offsets):
// blockIdx.x is the column tile, blockIdx.y walks the row tiles of the groups
// in order (group g: ceil(rows_g / BM) tiles; false past the last).  Dense: a
// 1-D grid of tiles_m x tiles_n tiles in the XCD-aware order.  Sets the group
// g, its row range [rb, re) and the tile (tm, tn).
template <int BM>
__device__ __forceinline__ bool dma_tile_coords(const TiledArgs& p, int tiles_m, int tiles_n, int& g,
                                                int64_t& rb, int64_t& re, int64_t& tm, int64_t& tn) {
    g = 0;
    rb = 0;
    re = p.m;
    if (p.offsets) {
        tn = blockIdx.x;
        int64_t t = blockIdx.y;
        auto bound = [&](int e) {
            return min(max(static_cast<int64_t>(p.offsets[e]), int64_t(0)), p.m);
        };
        g = -1;
        for (int e = 0; e < p.groups; ++e) {
            const int64_t rows = max(bound(e + 1) - bound(e), int64_t(0));
            const int64_t tiles = (rows + BM - 1) / BM;
            if (t < tiles) { g = e; break; }
            t -= tiles;
        }
        if (g < 0) return false;
        rb = bound(g);
        re = max(bound(g + 1), rb);
        tm = t;
    } else {
        // XCD-aware order: the dispatcher deals consecutive workgroup ids to
        // the XCDs in turn, so hand each XCD a contiguous run of tiles and
        // walk them in groups of 8 M-tiles (A and B tiles shared in one L2).
        const int64_t total = static_cast<int64_t>(tiles_m) * tiles_n;
        const int64_t i = blockIdx.x;
        const int64_t x = p.xcds;
        const int64_t full = total - total % x;
        int64_t L = i;
        if (i < full) L = (i % x) * (full / x) + i / x;
        constexpr int64_t kGroupM = 8;
        const int64_t group = L / (kGroupM * tiles_n);
        const int64_t first_m = group * kGroupM;
        const int64_t gsize = min(static_cast<int64_t>(tiles_m) - first_m, kGroupM);
        const int64_t in_group = L % (kGroupM * tiles_n);
        tm = first_m + in_group % gsize;
        tn = in_group / gsize;
    }
    return true;
}

// Store epilogue of one wave's (BM / 2) x (BN / (NW / 2)) block of a
// direct-to-LDS tile (wave (wm, wn) of the 2 x (NW / 2) wave grid), for every
// epilogue but the staged GLU one of the 64-k slab tile.  qkv_stage: this
// wave's own LDS region for the staged QKV epilogue (every wave calls this
// function: the staged path meets the others at a barrier first).
template <int BM, int BN, int NW, int EPI, bool PP, int WM, int WN>
__device__ __forceinline__ void dma_tile_epilogue(const TiledArgs& p, const floatx16 (&acc)[WM][WN], int wm,
                                                  int wn, int64_t row0, int64_t ncol0, int64_t re,
                                                  const float* scales, float* qkv_stage) {
    constexpr bool kGlu = EpiTraits<EPI>::glu;
    constexpr int kWavesM = 2, kWavesN = NW / 2;
    static_assert(WM == BM / (32 * kWavesM) && WN == BN / (32 * kWavesN), "wave block shape");
    // The epilogues take the lane index again from the lane mask, so no
    // lane-derived value of the prologue has to live through the main loop.
    const int elane = static_cast<int>(__lane_id());
    const int el32 = elane & 31, ekhalf = elane >> 5;
    // Epilogue: 32x32 D layout, lane holds column (lane & 31) and rows
    // 8 (r / 4) + 4 (lane >> 5) + (r % 4).  The output dtype and the scales are
    // resolved once per tile, a lane's scales (its columns are fixed) are read
    // once, and the residual loads of a group of half blocks (at clamped,
    // always valid addresses) all precede the group's first store, so the
    // group waits for memory once instead of once per element; only the
    // stores are guarded.
    if constexpr (EPI != kEpiQkvRope) {
        constexpr int kCols = kGlu ? WN / 2 : WN;  // output columns per lane
        int64_t cols[kCols];
        float sc_lo[kCols], sc_hi[kCols];
#pragma unroll
        for (int j = 0; j < kCols; ++j) {
            cols[j] = kGlu ? ncol0 + (wn * WN / 2 + j) * 32 + el32 : ncol0 + wn * (BN / kWavesN) + j * 32 + el32;
            const int64_t cc = min(cols[j], p.n - 1);
            sc_lo[j] = scales ? scales[cc] : 1.f;
            sc_hi[j] = (kGlu && scales) ? scales[p.n + cc] : 1.f;
        }
        // Residual rows [0, m) addressable with 32-bit byte offsets: loads go
        // through a buffer resource (reads past its end return 0, and every
        // load of a column >= n feeds only an output that is not stored).
        const bool res_rsrc_ok = EPI == SFG_EPI_RESIDUAL && p.residual &&
                                 static_cast<uint64_t>(p.m) * p.ldr * 4 <= 0xFFFFFFFFull;
        const buf_rsrc res_rsrc = make_rsrc(p.residual, res_rsrc_ok ? static_cast<uint32_t>(p.m * p.ldr * 4) : 0u);
        auto store_tile = [&](auto* out) {
            using OutT = std::remove_pointer_t<decltype(out)>;
            // Residual epilogues load the residual of kGroup half blocks before
            // the first of their stores (each element is still read before it
            // is written, so an in-place residual stays correct): the tile
            // waits for memory 2 WM / kGroup times instead of 2 WM.
            // (four-wave 256 x 256 tiles only: the others have no registers for it).
            constexpr int kGroup = (EPI == SFG_EPI_RESIDUAL && NW == 4 && BM == 256 && BN == 256) ? 4 : 1;
#pragma unroll
            for (int g0 = 0; g0 < 2 * WM; g0 += kGroup) {
                float res[kGroup][8][kCols];
                if constexpr (EPI == SFG_EPI_RESIDUAL) {
                    if (kGroup > 1 && res_rsrc_ok) {
                        // 32-bit offsets through a buffer resource over the
                        // residual rows [0, m): one offset per row, the column
                        // blocks 128 B apart as immediate offsets
#pragma unroll
                        for (int h = 0; h < kGroup; ++h) {
                            const int ih = g0 + h, i = ih >> 1, r0 = (ih & 1) * 8;
                            const int64_t rbase = row0 + wm * (BM / kWavesM) + i * 32 + 4 * ekhalf;
#pragma unroll
                            for (int rr = 0; rr < 8; ++rr) {
                                const int r = r0 + rr;
                                const int64_t row = min(rbase + 8 * (r >> 2) + (r & 3), re - 1);
                                const uint32_t off = static_cast<uint32_t>((row * p.ldr + cols[0]) * 4);
#pragma unroll
                                for (int j = 0; j < kCols; ++j)
                                    res[h][rr][j] = __builtin_bit_cast(
                                        float, __builtin_amdgcn_raw_buffer_load_b32(res_rsrc, off + j * 128, 0, 0));
                            }
                        }
                    } else {
#pragma unroll
                        for (int h = 0; h < kGroup; ++h) {
                            const int ih = g0 + h, i = ih >> 1, r0 = (ih & 1) * 8;
                            const int64_t rbase = row0 + wm * (BM / kWavesM) + i * 32 + 4 * ekhalf;
#pragma unroll
                            for (int rr = 0; rr < 8; ++rr)
#pragma unroll
                                for (int j = 0; j < kCols; ++j) {
                                    const int r = r0 + rr;
                                    const int64_t row = min(rbase + 8 * (r >> 2) + (r & 3), re - 1);
                                    res[h][rr][j] = p.residual[row * p.ldr + min(cols[j], p.n - 1)];
                                }
                        }
                    }
                }
#pragma unroll
                for (int h = 0; h < kGroup; ++h) {  // half 32-row blocks: 8 accumulator rows each
                    const int ih = g0 + h, i = ih >> 1, r0 = (ih & 1) * 8;
                    const int64_t rbase = row0 + wm * (BM / kWavesM) + i * 32 + 4 * ekhalf;
#pragma unroll
                    for (int rr = 0; rr < 8; ++rr) {
                        const int r = r0 + rr;
                        const int64_t row = rbase + 8 * (r >> 2) + (r & 3);
#pragma unroll
                        for (int j = 0; j < kCols; ++j) {
                            float v;
                            if constexpr (kGlu) {
                                v = glu_combine(EPI, acc[i][2 * j][r] * sc_lo[j], acc[i][2 * j + 1][r] * sc_hi[j]);
                            } else {
                                v = acc[i][j][r] * sc_lo[j];
                                if constexpr (EPI == SFG_EPI_RESIDUAL) v += res[h][rr][j];
                            }
                            if (row < re && cols[j] < p.n) {
                                if constexpr (sizeof(OutT) == 4) out[row * p.ldc + cols[j]] = v;
                                else out[row * p.ldc + cols[j]] = f32_to_bf16(v);
                            }
                        }
                    }
                }
            }
        };
        if (p.c_dtype == SFG_F32) store_tile(static_cast<float*>(p.c));
        else store_tile(static_cast<uint16_t*>(p.c));
    }
    if constexpr (EPI == kEpiQkvRope) {
        // four-wave tiles with square wave blocks stage through LDS (a wave's
        // own stage array holds its fp32 32-row block and its V^T block)
        constexpr bool kStaged = NW == 4 && !PP && ((WM == 4 && WN == 4) || (WM == 2 && WN == 2));
        if constexpr (kStaged) {
            // every wave's reads of the last slabs are done before any wave
            // reuses its array as staging (the DMA drained above)
            wait_lds();
            barrier_no_fence();
            qkv_rope_epilogue_staged<WM, WN>(p.qkv, acc, row0 + wm * (BM / kWavesM), ncol0 + wn * (BN / kWavesN),
                                             re, p.n, elane, qkv_stage);
        } else {
            qkv_rope_epilogue<WM, WN>(p.qkv, acc, row0 + wm * (BM / kWavesM), ncol0 + wn * (BN / kWavesN), re,
                                      p.n, el32, ekhalf);
        }
    }
}

template <int BM, int BN, int NW, int EPI, bool PP = false, bool S64 = false>
__global__ __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(DmaShapeTraits<BM, BN, NW>::occupancy,
                                   DmaShapeTraits<BM, BN, NW>::occupancy)))
void gemm_dma_kernel(TiledArgs p, int tiles_m, int tiles_n) {
    static_assert(!PP || (NW == 8 && DmaShapeTraits<BM, BN, NW>::stages == 4),
                  "ping-pong pairs two four-wave groups over a four-stage ring");
    static_assert(!S64 || (BM == 256 && BN == 256 && NW == 4 && !PP),
                  "the 64-k slab loop runs the four-wave 256 x 256 tile");
    constexpr bool kGlu = EpiTraits<EPI>::glu;
    constexpr int kStages = DmaShapeTraits<BM, BN, NW>::stages;
    constexpr int kWavesM = 2, kWavesN = NW / 2;
    constexpr int WM = BM / (32 * kWavesM), WN = BN / (32 * kWavesN);  // 32x32 tiles per wave
    constexpr int kDmaBytes = DmaShapeTraits<BM, BN, NW>::dma_bytes;   // per lane per DMA instruction
    constexpr int kDmaRows = kDmaBytes;                                 // 64-byte rows per instruction
    constexpr int kLoadsA = BM / kDmaRows / NW, kLoadsB = BN / kDmaRows / NW;  // DMA instructions per wave per slab
    constexpr int kLoads = kLoadsA + kLoadsB;
    static_assert(!kGlu || WN % 2 == 0, "GLU tiles pair gate and up blocks");
    __shared__ __attribute__((aligned(1024))) uint16_t sS0[(BM + BN) * kRK];
    __shared__ __attribute__((aligned(1024))) uint16_t sS1[(BM + BN) * kRK];
    __shared__ __attribute__((aligned(1024))) uint16_t sS2[(BM + BN) * kRK];
    __shared__ __attribute__((aligned(1024))) uint16_t sS3[(BM + BN) * kRK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS addresses in SGPRs
    const int wm = wave / kWavesN, wn = wave % kWavesN;
    constexpr int kOutCols = kGlu ? BN / 2 : BN;

    int g;
    int64_t rb, re, tm, tn;
    if (!dma_tile_coords<BM>(p, tiles_m, tiles_n, g, rb, re, tm, tn)) return;
    const int64_t row0 = rb + tm * BM;
    if (row0 >= re) return;
    const int64_t ncol0 = tn * kOutCols;
    const int64_t bgroup = static_cast<int64_t>(g) * p.b_group_stride;
    const float* scales = p.scales ? p.scales + static_cast<int64_t>(g) * p.s_group_stride : nullptr;

    // Load assignment: wave instruction i fills block (i * NW + wave); lane l
    // covers row 16 * block + (l >> 2) and destination slot (l & 3), fetching
    // the chunk (l & 3) ^ ((row >> 2) & 3).  Rows past the tile's end read a
    // valid row instead (their results are never stored).
    // The loads go through buffer resources over A and over this group's B
    // (byte offsets; the host guarantees both fit 32 bits).
    // One DMA instruction fills kDmaRows rows of 64 B (kDmaBytes per lane):
    // lane l covers row l / (64 / kDmaBytes) of its block and the 16-byte
    // destination slot s it lands in holds global chunk s ^ ((row >> 2) & 3).
    constexpr int kLanesPerRow = 64 / kDmaBytes;
    const int lrow = lane / kLanesPerRow;
    const int piece = lane % kLanesPerRow;
    const int slot16 = piece * kDmaBytes / 16;
    const int sub = (piece % (16 / kDmaBytes)) * (kDmaBytes / 2);  // bf16 offset inside the 16-byte slot
    auto chunk_of = [&](int local_row) { return ((slot16 ^ ((local_row >> 2) & 3)) * 8) + sub; };
    // A gathered id outside [0, a_rows_limit) is a zero row: its loads start
    // at the end of A's resource, so every slab of it reads the zeros an
    // out-of-range buffer load returns (the host keeps that offset plus any
    // k offset inside 32 bits).
    const uint32_t a_bytes = static_cast<uint32_t>(p.a_rows_limit * p.lda * 2);
    const buf_rsrc ra = make_rsrc(p.a, a_bytes);
    uint32_t a_off[kLoadsA];
#pragma unroll
    for (int i = 0; i < kLoadsA; ++i) {
        const int local = (i * NW + wave) * kDmaRows + lrow;
        const int64_t r = row0 + local;
        int64_t src = r < re ? r : row0;
        if (p.a_rows) src = p.a_rows[src];
        a_off[i] = (src < 0 || src >= p.a_rows_limit) ? a_bytes
                                                      : static_cast<uint32_t>((src * p.lda + chunk_of(local)) * 2);
    }
    const uint16_t* bbase = static_cast<const uint16_t*>(p.b) + bgroup;
    const buf_rsrc rb_ = make_rsrc(bbase, static_cast<uint32_t>((kGlu ? 2 : 1) * p.n * p.ldb * 2));
    uint32_t b_off[kLoadsB];
#pragma unroll
    for (int i = 0; i < kLoadsB; ++i) {
        const int local = (i * NW + wave) * kDmaRows + lrow;
        int64_t brow;
        if (kGlu) {
            const int block = local >> 5;
            const int64_t col = ncol0 + (block >> 1) * 32 + (local & 31);
            brow = col < p.n ? ((block & 1) ? p.n + col : col) : 0;
        } else {
            const int64_t col = ncol0 + local;
            brow = col < p.n ? col : 0;
        }
        b_off[i] = static_cast<uint32_t>((brow * p.ldb + chunk_of(local)) * 2);
    }

    auto issue = [&](uint16_t* da, int64_t k0) {
        uint16_t* db = da + BM * kRK;
        const uint32_t kb = static_cast<uint32_t>(k0 * 2);
#pragma unroll
        for (int i = 0; i < kLoadsA; ++i)
            lds_dma_buf<kDmaBytes>(ra, a_off[i], kb, da + (i * NW + wave) * kDmaRows * kRK);
#pragma unroll
        for (int i = 0; i < kLoadsB; ++i)
            lds_dma_buf<kDmaBytes>(rb_, b_off[i], kb, db + (i * NW + wave) * kDmaRows * kRK);
    };

    floatx16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int l32 = lane & 31;
    const int khalf = lane >> 5;
    const int swz = (l32 >> 2) & 3;  // == (row >> 2) & 3 for every fragment row this lane reads
    // Fragments of one 16-k step: A tiles WM, B tiles WN.
    auto load_frags = [&](const uint16_t* S, int kk, bf16x8* fa, bf16x8* fb) {
        const uint16_t* A = S;
        const uint16_t* B = S + BM * kRK;
        const int slot = ((kk * 2 + khalf) ^ swz) * 8;
#pragma unroll
        for (int i = 0; i < WM; ++i)
            fa[i] = as_bf16x8(*reinterpret_cast<const uint4*>(&A[(wm * (BM / kWavesM) + i * 32 + l32) * kRK + slot]));
#pragma unroll
        for (int j = 0; j < WN; ++j)
            fb[j] = as_bf16x8(*reinterpret_cast<const uint4*>(&B[(wn * (BN / kWavesN) + j * 32 + l32) * kRK + slot]));
    };
    auto mfmas = [&](const bf16x8* fa, const bf16x8* fb) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    };

    // Ring of kStages stages, software-pipelined one half-slab ahead.  Slab kt
    // (stage cur) runs as
    //   read the k-step-1 fragments of slab kt     | MFMAs of k-step 0
    //   issue slab kt + kStages - 1 into the stage slab kt - 1 used
    //   wait for this wave's loads of slab kt + 1 and its fragment reads, barrier
    //   read the k-step-0 fragments of slab kt + 1 | MFMAs of k-step 1
    // so every LDS read overlaps WM x WN MFMAs, and the barrier that publishes
    // slab kt + 1 also retires every read of stage cur before a later issue
    // overwrites it.  The issue sits right before the wait: the compiler counts
    // an LDS DMA as a pending FLAT access on lgkmcnt and, while one is pending,
    // waits for lgkmcnt(0) before using any fragment; the wait's lgkmcnt(0)
    // retires it, so the fragment reads after the barrier get partial waits.
    // Every slab issues exactly one load group (past
    // the end it re-fetches the last slab into a stage nobody reads again), so
    // the wait is always "all but the kStages - 2 newest groups" and the
    // compiler's LDS-DMA tracking sees one uniform pattern (with conditional
    // issues it waits for every load before the fragment reads).  The loop is
    // unrolled by kStages so every stage is a fixed __shared__ array.
    const int64_t slabs = p.k / kRK;
    bf16x8 f0a[WM], f0b[WN], f1a[WM], f1b[WN];
    auto slab = [&](int64_t kt, const uint16_t* cur, uint16_t* prev, const uint16_t* next) {
        load_frags(cur, 1, f1a, f1b);
        __builtin_amdgcn_sched_barrier(0);
        if (kt < slabs) mfmas(f0a, f0b);
        __builtin_amdgcn_sched_barrier(0);
        issue(prev, min(kt + kStages - 1, slabs - 1) * kRK);
        wait_vmem_lds<(kStages - 2) * kLoads>();
        barrier_no_fence();
        load_frags(next, 0, f0a, f0b);
        __builtin_amdgcn_sched_barrier(0);
        if (kt < slabs) mfmas(f1a, f1b);
        __builtin_amdgcn_sched_barrier(0);
    };
    // The same slab for kt < slabs with its instructions interleaved: each
    // half runs its MFMAs one by one with the next half's fragment reads and
    // (first half) the slab's DMA issues placed between them, so a wave that
    // is alone on its SIMD keeps the matrix pipe fed while it reads LDS and
    // issues loads, and reaches the barrier with only its last MFMA in flight.
    auto slab_il = [&](int64_t kt, const uint16_t* cur, uint16_t* prev, const uint16_t* next) {
        load_frags(cur, 1, f1a, f1b);
        mfmas(f0a, f0b);
        issue(prev, min(kt + kStages - 1, slabs - 1) * kRK);
        interleave_groups<WM * WN, WM + WN, kLoads>();
        __builtin_amdgcn_sched_barrier(0);
        wait_vmem_lds<(kStages - 2) * kLoads>();
        barrier_no_fence();
        load_frags(next, 0, f0a, f0b);
        mfmas(f1a, f1b);
        interleave_groups<WM * WN, WM + WN, 0>();
        __builtin_amdgcn_sched_barrier(0);
    };
    if constexpr (S64) {
        // 64-k slabs, one barrier per slab.  Each wave owns 128 x 128 of the
        // tile (4 x 4 MFMA tiles, accumulators in AGPRs).  Both operands go
        // global -> LDS by DMA, A into a two-stage ring (sS0, sS2) and B into a
        // three-stage ring (sS1, sS3, sS4): the whole 160 KB.  LDS rows are
        // 128 B with chunk c of row r in slot c ^ ((r >> 1) & 7), so the 16
        // lanes of one ds_read_b128 pass touch 16 distinct 16-byte bank
        // groups; a DMA instruction fills 8 rows (lane l: row l >> 3, slot
        // l & 7), each lane fetching the global chunk its slot holds.
        //   B of slab s + 2 is issued during k-steps 0..2 of slab s into the
        //   stage slab s - 1 used (free since the barrier that ended it);
        //   A of slab s + 2 can go only into the stage slab s uses, so half of
        //   it is issued right after slab s's barrier and half under the next
        //   slab's first k-step.
        // Slab s runs four 16-k steps of 16 MFMAs; under each the wave reads
        // the next step's 8 fragments and issues its share of DMA.  Two MFMAs
        // into k-step 3 it waits for its own DMA of slab s + 1 (all but the 8 B
        // instructions of slab s + 2, which are the newest) and its LDS reads,
        // meets the other waves at the barrier, and reads slab s + 1's first
        // fragments under the remaining 14 MFMAs.  Every slab issues the same
        // DMA pattern (past the end it re-fetches the last slab into a free
        // stage), so the vmcnt accounting is uniform.
        __shared__ __attribute__((aligned(1024))) uint16_t sS4[(BM + BN) * kRK];
        constexpr int kBK = 64;
        constexpr int kRowB = kBK * 2;        // bytes per LDS row
        constexpr int kRows32 = 32 * kRowB;   // bytes of 32 rows
        constexpr int kPre = 2;               // MFMAs of k-step 3 before the barrier
        const int64_t nslab = p.k / kBK;
        // DMA instruction i (< 8) of this wave fills rows (4 i + wave) * 8 ..+8
        uint32_t dma_a[8], dma_b[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int local = (4 * i + wave) * 8 + (lane >> 3);
            const int chunk = (lane & 7) ^ ((local >> 1) & 7);
            const int64_t r = row0 + local;
            int64_t src = r < re ? r : row0;
            if (p.a_rows) src = p.a_rows[src];
            dma_a[i] = (src < 0 || src >= p.a_rows_limit) ? a_bytes  // zero row, as above
                                                          : static_cast<uint32_t>((src * p.lda + chunk * 8) * 2);
            int64_t brow;
            if (kGlu) {
                const int block = local >> 5;
                const int64_t col = ncol0 + (block >> 1) * 32 + (local & 31);
                brow = col < p.n ? ((block & 1) ? p.n + col : col) : 0;
            } else {
                const int64_t col = ncol0 + local;
                brow = col < p.n ? col : 0;
            }
            dma_b[i] = static_cast<uint32_t>((brow * p.ldb + chunk * 8) * 2);
        }
        const int fsw = (l32 >> 1) & 7;
        uint32_t ra_off[4], rb_off[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ra_off[j] = static_cast<uint32_t>((wm * 128 + l32) * kRowB + (((2 * j + khalf) ^ fsw) * 16));
            rb_off[j] = static_cast<uint32_t>((wn * 128 + l32) * kRowB + (((2 * j + khalf) ^ fsw) * 16));
        }
        char* const stA[2] = {reinterpret_cast<char*>(sS0), reinterpret_cast<char*>(sS2)};
        char* const stB[3] = {reinterpret_cast<char*>(sS1), reinterpret_cast<char*>(sS3),
                              reinterpret_cast<char*>(sS4)};
        auto dma = [&](char* const* stages, const buf_rsrc& rs, const uint32_t (&off)[8], int st,
                       int64_t kt, int i0, int i1) {
            const uint32_t soff = static_cast<uint32_t>(min(kt, nslab - 1) * kBK * 2);
#pragma unroll
            for (int i = i0; i < i1; ++i)
                lds_dma16_buf(rs, off[i], soff, reinterpret_cast<uint16_t*>(stages[st] + (4 * i + wave) * 8 * kRowB));
        };
        auto dma_A = [&](int st, int64_t kt, int i0, int i1) { dma(stA, ra, dma_a, st, kt, i0, i1); };
        auto dma_B = [&](int st, int64_t kt, int i0, int i1) { dma(stB, rb_, dma_b, st, kt, i0, i1); };
        bf16x8 fa[2][4], fb[2][4];
        // in the order the row-major MFMAs consume them: a0, b0..b3, a1..a3
        auto frags = [&](int sa, int sb, int j, bf16x8 (&a)[4], bf16x8 (&b)[4]) {
            a[0] = as_bf16x8(*reinterpret_cast<const uint4*>(stA[sa] + ra_off[j]));
#pragma unroll
            for (int i = 0; i < 4; ++i)
                b[i] = as_bf16x8(*reinterpret_cast<const uint4*>(stB[sb] + rb_off[j] + i * kRows32));
#pragma unroll
            for (int i = 1; i < 4; ++i)
                a[i] = as_bf16x8(*reinterpret_cast<const uint4*>(stA[sa] + ra_off[j] + i * kRows32));
        };
        // MFMAs q0 .. q1 - 1 of a k-step, row-major over the 4 x 4 tiles
        auto mfmas = [&](const bf16x8 (&a)[4], const bf16x8 (&b)[4], int q0, int q1) {
#pragma unroll
            for (int q = q0; q < q1; ++q)
                acc[q / 4][q % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[q / 4], b[q % 4], acc[q / 4][q % 4], 0, 0, 0);
        };
        // Slab s (s % 6 == C): A stage s % 2, B stage s % 3.
        auto slab64 = [&](int64_t s, auto c_c) {
            constexpr int C = decltype(c_c)::value;
            constexpr int sa = C % 2, sb = C % 3, nb = (sb + 2) % 3;
            frags(sa, sb, 1, fa[1], fb[1]);
            dma_A(sa ^ 1, s + 1, 4, 8);  // second half of A's slab s + 1
            mfmas(fa[0], fb[0], 0, 4);
            spread_reads_loads<4, 4, 4>();
            __builtin_amdgcn_sched_barrier(0);
            // every A instruction of slab s + 1 precedes every B one of slab s + 2
            dma_B(nb, s + 2, 0, 3);
            mfmas(fa[0], fb[0], 4, 16);
            spread_reads_loads<12, 4, 3>();
            __builtin_amdgcn_sched_barrier(0);
            frags(sa, sb, 2, fa[0], fb[0]);
            dma_B(nb, s + 2, 3, 6);
            mfmas(fa[1], fb[1], 0, 16);
            spread_reads_loads<16, 8, 3>();
            __builtin_amdgcn_sched_barrier(0);
            frags(sa, sb, 3, fa[1], fb[1]);
            dma_B(nb, s + 2, 6, 8);
            mfmas(fa[0], fb[0], 0, 16);
            spread_reads_loads<16, 8, 2>();
            __builtin_amdgcn_sched_barrier(0);
            mfmas(fa[1], fb[1], 0, kPre);
            __builtin_amdgcn_sched_barrier(0);
            wait_vmem_lds<8>();
            barrier_no_fence();
            dma_A(sa, s + 2, 0, 4);      // first half of A's slab s + 2
            frags(sa ^ 1, (sb + 1) % 3, 0, fa[0], fb[0]);
            mfmas(fa[1], fb[1], kPre, 16);
            spread_reads_loads<16 - kPre, 8, 4>();
            __builtin_amdgcn_sched_barrier(0);
        };
        // prologue: A and B of slab 0, B of slab 1, then the first half of A's slab 1
        dma_A(0, 0, 0, 8);
        dma_B(0, 0, 0, 8);
        dma_B(1, 1, 0, 8);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmem_lds<8>();
        barrier_no_fence();
        dma_A(1, 1, 0, 4);
        frags(0, 0, 0, fa[0], fb[0]);
        using c0 = std::integral_constant<int, 0>;
        using c1 = std::integral_constant<int, 1>;
        using c2 = std::integral_constant<int, 2>;
        using c3 = std::integral_constant<int, 3>;
        using c4 = std::integral_constant<int, 4>;
        using c5 = std::integral_constant<int, 5>;
        // unrolled by 6 (stage periods 2 and 3), so every stage is a fixed array
        int64_t s = 0;
        for (; s + 6 <= nslab; s += 6) {
            slab64(s, c0{});
            slab64(s + 1, c1{});
            slab64(s + 2, c2{});
            slab64(s + 3, c3{});
            slab64(s + 4, c4{});
            slab64(s + 5, c5{});
        }
        if (s < nslab) slab64(s, c0{});
        if (s + 1 < nslab) slab64(s + 1, c1{});
        if (s + 2 < nslab) slab64(s + 2, c2{});
        if (s + 3 < nslab) slab64(s + 3, c3{});
        if (s + 4 < nslab) slab64(s + 4, c4{});
    } else {
    issue(sS0, 0);
    issue(sS1, min(int64_t(1), slabs - 1) * kRK);
    if constexpr (kStages == 4) issue(sS2, min(int64_t(2), slabs - 1) * kRK);
    wait_vmem_lds<(kStages - 2) * kLoads>();
    barrier_no_fence();
    if constexpr (PP) {
        // Ping-pong: waves 0..3 (one per SIMD) lead, waves 4..7 trail by one
        // phase; between consecutive barriers one group multiplies a whole
        // slab while the other reads the next slab's fragments and issues its
        // loads, so each SIMD's MFMA pipe always has one group feeding it.
        //   leader:  mem(0) | mul(0) | mem(1) | mul(1) | ... | (idle)
        //   trailer: (idle) | mem(0) | mul(0) | mem(1) | ... | mul(last)
        // mem(s) reads both k-steps of slab s, issues slab s + 3 into the stage
        // slab s - 1 used, waits for its own loads of slab s + 1 and its reads.
        // Every read of a slab is retired (lgkmcnt(0)) before a barrier that
        // precedes the next issue into its stage, and every wave's loads of
        // slab s + 1 are complete before the barrier that precedes the first
        // read of slab s + 1 (by the leader, one phase before the trailer).
        auto mem = [&](int64_t kt, const uint16_t* cur, uint16_t* prev) {
            load_frags(cur, 0, f0a, f0b);
            load_frags(cur, 1, f1a, f1b);
            issue(prev, min(kt + kStages - 1, slabs - 1) * kRK);
            wait_vmem_lds<(kStages - 2) * kLoads>();
            barrier_no_fence();
        };
        auto mul = [&](int64_t kt) {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
            if (kt < slabs) {
                mfmas(f0a, f0b);
                mfmas(f1a, f1b);
            }
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            barrier_no_fence();
        };
        const bool trailer = wave >= NW / 2;
        if (trailer) barrier_no_fence();
        for (int64_t kt = 0; kt < slabs; kt += 4) {
            mem(kt, sS0, sS3);
            mul(kt);
            mem(kt + 1, sS1, sS0);
            mul(kt + 1);
            mem(kt + 2, sS2, sS1);
            mul(kt + 2);
            mem(kt + 3, sS3, sS2);
            mul(kt + 3);
        }
        if (!trailer) barrier_no_fence();
    } else {
    if constexpr (DmaShapeTraits<BM, BN, NW>::slab_ahead) {
        // A whole slab ahead in registers.  The MFMAs of slab kt use fragments
        // read during slab kt - 1; while they run, the wave reads slab kt + 1
        // from LDS into the other register set and issues slab kt + 4 into the
        // stage slab kt occupied (every wave finished reading it before the
        // barrier that opened slab kt).  One wait + barrier per slab, at its
        // end: slab kt + 2 must have landed (kt + 3 and kt + 4 stay in flight)
        // and this wave's reads of slab kt + 1 must be done; after it the next
        // MFMAs start at once, their operands already in registers.
        issue(sS3, min(int64_t(3), slabs - 1) * kRK);
        bf16x8 ga[2][2][WM], gb[2][2][WN];  // [register set][k-step][fragment]
        load_frags(sS0, 0, ga[0][0], gb[0][0]);
        load_frags(sS0, 1, ga[0][1], gb[0][1]);
        wait_vmem_lds<2 * kLoads>();
        barrier_no_fence();
        auto step = [&](int64_t kt, auto set_c, const uint16_t* next_stage, uint16_t* own_stage, bool live) {
            constexpr int c = decltype(set_c)::value, n = 1 - c;
            load_frags(next_stage, 0, ga[n][0], gb[n][0]);
            if (live) mfmas(ga[c][0], gb[c][0]);
            issue(own_stage, min(kt + 4, slabs - 1) * kRK);
            interleave_groups<WM * WN, WM + WN, kLoads>();
            __builtin_amdgcn_sched_barrier(0);
            load_frags(next_stage, 1, ga[n][1], gb[n][1]);
            if (live) mfmas(ga[c][1], gb[c][1]);
            interleave_groups<WM * WN, WM + WN, 0>();
            __builtin_amdgcn_sched_barrier(0);
            wait_vmem_lds<2 * kLoads>();
            barrier_no_fence();
        };
        using set0 = std::integral_constant<int, 0>;
        using set1 = std::integral_constant<int, 1>;
        int64_t kt = 0;
        for (; kt + 4 <= slabs; kt += 4) {
            step(kt, set0{}, sS1, sS0, true);
            step(kt + 1, set1{}, sS2, sS1, true);
            step(kt + 2, set0{}, sS3, sS2, true);
            step(kt + 3, set1{}, sS0, sS3, true);
        }
        if (kt < slabs) {
            step(kt, set0{}, sS1, sS0, kt < slabs);
            step(kt + 1, set1{}, sS2, sS1, kt + 1 < slabs);
            step(kt + 2, set0{}, sS3, sS2, kt + 2 < slabs);
        }
    } else {
    load_frags(sS0, 0, f0a, f0b);
    if constexpr (kStages == 4) {
        // whole groups of four slabs interleaved, then at most one guarded group
        int64_t kt = 0;
        for (; kt + 4 <= slabs; kt += 4) {
            slab_il(kt, sS0, sS3, sS1);
            slab_il(kt + 1, sS1, sS0, sS2);
            slab_il(kt + 2, sS2, sS1, sS3);
            slab_il(kt + 3, sS3, sS2, sS0);
        }
        if (kt < slabs) {
            slab(kt, sS0, sS3, sS1);
            slab(kt + 1, sS1, sS0, sS2);
            slab(kt + 2, sS2, sS1, sS3);
            slab(kt + 3, sS3, sS2, sS0);
        }
    } else {
        for (int64_t kt = 0; kt < slabs; kt += 3) {
            slab(kt, sS0, sS2, sS1);
            slab(kt + 1, sS1, sS0, sS2);
            slab(kt + 2, sS2, sS1, sS0);
        }
    }
    }
    }
    }
    wait_vmem<0>();

    if constexpr (S64 && kGlu) {
        if (p.c_dtype == SFG_BF16) {
            // the lane index again from the lane mask, so no lane-derived
            // value of the prologue has to live through the main loop
            const int elane = static_cast<int>(__lane_id());
            // every wave's reads of the last slabs are done before any wave
            // reuses its array as staging (the DMA drained above)
            wait_lds();
            barrier_no_fence();
            uint16_t* const stage = wave == 0 ? sS0 : wave == 1 ? sS1 : wave == 2 ? sS2 : sS3;
            glu_epilogue_staged<EPI>(p, acc, row0 + wm * (BM / kWavesM), ncol0 + wn * (BN / 4), re, scales,
                                     elane, stage);
            return;
        }
    }

    float* const qkv_stage = reinterpret_cast<float*>(wave == 0 ? sS0 : wave == 1 ? sS1 : wave == 2 ? sS2 : sS3);
    dma_tile_epilogue<BM, BN, NW, EPI, PP>(p, acc, wm, wn, row0, ncol0, re, scales, qkv_stage);
}

// ===========================================================================
// VALU GEMM: 64x64, 32x32, 16x32 or 16x16 tiles (k slabs of 16 to 128),
// 256 threads, one fp32 FMA chain per output in k order.  The fp32 path (AT = BT = float), and
// the fallback for bf16 / int8 products the MFMA kernels do not lower (K not a
// multiple of their k step, rows not 16-byte aligned): A fp32 or bf16, B fp32,
// bf16 or int8 with per-channel scales applied after the sum; grouped
// problems and the dispatch gather as in the tiled kernels.
// For GLU epilogues a thread's columns are RN / 2 of the gate block and the
// same RN / 2 of the up block.
// ===========================================================================
struct VecArgs {
    const void* a; int64_t lda; const int32_t* a_rows; int64_t a_rows_limit;
    const void* b; int64_t ldb; const float* scales;
    int64_t b_group_stride, s_group_stride;
    void* c; int c_dtype; int64_t ldc;
    const float* residual; int64_t ldr;
    int64_t m, n, k;
    const int32_t* offsets; int groups;
};

template <typename T>
__device__ __forceinline__ float elem_f32(const T* p, int64_t i) {
    if constexpr (std::is_same_v<T, float>) return p[i];
    else if constexpr (std::is_same_v<T, int8_t>) return static_cast<float>(p[i]);
    else return bf16_to_f32(p[i]);
}

constexpr int kVecMinTiles = 256;  // VALU GEMM: smallest grid a tile may give

// TM x TN output tile per workgroup of 16 x 16 threads, RM x RN outputs per
// thread (TM = 16 RM, TN = 16 RN B rows; GLU tiles hold TN / 2 gate and TN / 2
// up rows and give TN / 2 output columns).  Every output is one sequential
// fp32 FMA chain over k whatever the tile, so every tile gives the same bits.
template <typename AT, typename BT, int EPI, int TM, int TN, int KS>
__global__ __launch_bounds__(256) void gemm_vec_kernel(VecArgs p) {
    constexpr bool kGlu = EpiTraits<EPI>::glu;
    constexpr int RM = TM / 16, RN = TN / 16;
    static_assert(TM % 16 == 0 && TN % 16 == 0, "tiles of 16 x 16 threads");
    static_assert(!kGlu || RN % 2 == 0, "GLU threads pair gate and up columns");
    // KS: k per LDS slab; each thread moves LA elements of A and LB of B per slab
    static_assert(KS >= 16 && KS <= 256 && (KS & (KS - 1)) == 0, "slab depth");
    constexpr int kKsShift = KS == 16 ? 4 : KS == 32 ? 5 : KS == 64 ? 6 : KS == 128 ? 7 : 8;
    constexpr int LA = TM * KS / 256, LB = TN * KS / 256;
    static_assert(LA >= 1 && LB >= 1, "every thread moves A and B elements");
    __shared__ float sA[2][KS][TM + 4];
    __shared__ float sB[2][KS][TN + 4];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    // Map blockIdx.y to (group, row tile).
    int g = 0;
    int64_t rb = 0, re = p.m, mtile = blockIdx.y;
    if (p.offsets) {
        int64_t t = blockIdx.y;
        g = -1;
        auto bound = [&](int e) { return min(max(static_cast<int64_t>(p.offsets[e]), int64_t(0)), p.m); };
        for (int e = 0; e < p.groups; ++e) {
            const int64_t lo = bound(e);
            const int64_t tiles = (max(bound(e + 1) - lo, int64_t(0)) + TM - 1) / TM;
            if (t < tiles) { g = e; break; }
            t -= tiles;
        }
        if (g < 0) return;
        rb = bound(g);
        re = max(bound(g + 1), rb);
        mtile = t;
    }
    const int64_t m0 = rb + mtile * TM;
    if (m0 >= re) return;
    const AT* A = static_cast<const AT*>(p.a);
    const BT* B = static_cast<const BT*>(p.b) + static_cast<int64_t>(g) * p.b_group_stride;
    const float* scales = p.scales ? p.scales + static_cast<int64_t>(g) * p.s_group_stride : nullptr;
    constexpr int kOutCols = kGlu ? TN / 2 : TN;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kOutCols;
    // B tile row -> B matrix row; valid when its output column is below n.
    auto brow_of = [&](int local) -> int64_t {
        if (kGlu) return local < TN / 2 ? n0 + local : p.n + n0 + local - TN / 2;
        return n0 + local;
    };
    auto bcol_ok = [&](int local) -> bool {
        return kGlu ? (local < TN / 2 ? n0 + local : n0 + local - TN / 2) < p.n : n0 + local < p.n;
    };
    float acc[RM][RN] = {};
    // this thread's RN B-tile rows: GLU, RN / 2 gate rows and the matching up rows
    int bc[RN];
#pragma unroll
    for (int j = 0; j < RN; ++j) {
        if (kGlu) bc[j] = (j < RN / 2) ? (RN / 2) * tx + j : TN / 2 + (RN / 2) * tx + (j - RN / 2);
        else bc[j] = RN * tx + j;
    }
    // This thread moves elements e = tid + 256 i of each TM x KS slab of A
    // (i < LA) and TN x KS slab of B (i < LB): row e / KS, k e % KS (the same
    // k for every i).  Sources are resolved once (the dispatch gather
    // included); -1 marks a row past the tile, which loads 0.
    const int lk = tid & (KS - 1);
    int64_t a_src[LA], b_src[LB];
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int r = (tid + 256 * i) >> kKsShift;
        const int64_t gr = m0 + r;
        int64_t src = -1;
        if (gr < re) {
            src = p.a_rows ? p.a_rows[gr] : gr;
            if (src < 0 || src >= p.a_rows_limit) src = -1;
        }
        a_src[i] = src < 0 ? -1 : src * p.lda;
    }
#pragma unroll
    for (int i = 0; i < LB; ++i) {
        const int r = (tid + 256 * i) >> kKsShift;
        b_src[i] = bcol_ok(r) ? brow_of(r) * p.ldb : -1;
    }
    // Two LDS stages: slab s + 1 is loaded into registers while slab s is
    // multiplied, then stored into the other stage (one barrier per slab).
    float va[LA], vb[LB];
    auto fetch = [&](int64_t k0) {
        const int64_t gk = k0 + lk;
        const bool kin = gk < p.k;
#pragma unroll
        for (int i = 0; i < LA; ++i) va[i] = (kin && a_src[i] >= 0) ? elem_f32(A, a_src[i] + gk) : 0.f;
#pragma unroll
        for (int i = 0; i < LB; ++i) vb[i] = (kin && b_src[i] >= 0) ? elem_f32(B, b_src[i] + gk) : 0.f;
    };
    auto stash = [&](int st) {
#pragma unroll
        for (int i = 0; i < LA; ++i) sA[st][lk][(tid + 256 * i) >> kKsShift] = va[i];
#pragma unroll
        for (int i = 0; i < LB; ++i) sB[st][lk][(tid + 256 * i) >> kKsShift] = vb[i];
    };
    fetch(0);
    stash(0);
    __syncthreads();
    int st = 0;
    for (int64_t k0 = 0; k0 < p.k; k0 += KS, st ^= 1) {
        const bool more = k0 + KS < p.k;
        if (more) fetch(k0 + KS);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            float av[RM], bv[RN];
#pragma unroll
            for (int i = 0; i < RM; ++i) av[i] = sA[st][kk][ty * RM + i];
#pragma unroll
            for (int j = 0; j < RN; ++j) bv[j] = sB[st][kk][bc[j]];
#pragma unroll
            for (int i = 0; i < RM; ++i)
#pragma unroll
                for (int j = 0; j < RN; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        // the other stage was last read before the previous barrier
        if (more) stash(st ^ 1);
        __syncthreads();
    }
    // per-channel scales of int8 weights (quantized_invoke, next_milestones.cpp:50-69)
    float sc[RN];
#pragma unroll
    for (int j = 0; j < RN; ++j) sc[j] = (scales && bcol_ok(bc[j])) ? scales[brow_of(bc[j])] : 1.f;
#pragma unroll
    for (int i = 0; i < RM; ++i) {
        const int64_t row = m0 + ty * RM + i;
        if (row >= re) continue;
        if (kGlu) {
#pragma unroll
            for (int j = 0; j < RN / 2; ++j) {
                const int64_t col = n0 + bc[j];
                if (col < p.n)
                    store_out(p.c, p.c_dtype, row * p.ldc + col,
                              glu_combine(EPI, acc[i][j] * sc[j], acc[i][j + RN / 2] * sc[j + RN / 2]));
            }
        } else {
#pragma unroll
            for (int j = 0; j < RN; ++j) {
                const int64_t col = n0 + bc[j];
                if (col >= p.n) continue;
                float v = acc[i][j] * sc[j];
                if (EPI == SFG_EPI_RESIDUAL) v += p.residual[row * p.ldr + col];
                store_out(p.c, p.c_dtype, row * p.ldc + col, v);
            }
        }
    }
}

template <typename AT, typename BT, int TM, int TN, int KS>
void launch_vec_tile(const VecArgs& a, int epi, hipStream_t stream) {
    const bool glu = epi == SFG_EPI_SWIGLU || epi == SFG_EPI_GLU_SILU_UP;
    const int64_t cols = glu ? TN / 2 : TN;
    const int64_t row_tiles = a.offsets ? (a.m + TM - 1) / TM + a.groups : (a.m + TM - 1) / TM;
    const dim3 grid(static_cast<unsigned>((a.n + cols - 1) / cols), static_cast<unsigned>(row_tiles));
    switch (epi) {
        case SFG_EPI_NONE: gemm_vec_kernel<AT, BT, SFG_EPI_NONE, TM, TN, KS><<<grid, 256, 0, stream>>>(a); break;
        case SFG_EPI_RESIDUAL: gemm_vec_kernel<AT, BT, SFG_EPI_RESIDUAL, TM, TN, KS><<<grid, 256, 0, stream>>>(a); break;
        default:
            // GLU tiles pair gate and up rows per thread (the caller never
            // sends a GLU product to a one-column tile)
            if constexpr ((TN / 16) % 2 == 0) {
                if (epi == SFG_EPI_SWIGLU) gemm_vec_kernel<AT, BT, SFG_EPI_SWIGLU, TM, TN, KS><<<grid, 256, 0, stream>>>(a);
                else gemm_vec_kernel<AT, BT, SFG_EPI_GLU_SILU_UP, TM, TN, KS><<<grid, 256, 0, stream>>>(a);
            }
            break;
    }
}

// Largest tile that still gives a workgroup to most CUs: each thread's RM x RN
// chains run the whole K, so on small products (the fp32 parity config's 128
// rows) a 64 x 64 tile leaves most of the GPU idle with 16 chains per thread.
template <typename AT, typename BT>
void launch_vec_t(const VecArgs& a, int epi, hipStream_t stream) {
    const bool glu = epi == SFG_EPI_SWIGLU || epi == SFG_EPI_GLU_SILU_UP;
    auto tiles = [&](int64_t tm, int64_t tn) {
        const int64_t cols = glu ? tn / 2 : tn;
        return ((a.m + tm - 1) / tm + (a.offsets ? a.groups : 0)) * ((a.n + cols - 1) / cols);
    };
    // slab depth grows as the tile shrinks: each thread keeps moving 4 - 8
    // elements per slab, so a slab's loads cover its chain steps' latency
    if (tiles(64, 64) >= kVecMinTiles) launch_vec_tile<AT, BT, 64, 64, 16>(a, epi, stream);
    else if (tiles(32, 32) >= kVecMinTiles) launch_vec_tile<AT, BT, 32, 32, 32>(a, epi, stream);
    else if (glu) launch_vec_tile<AT, BT, 16, 32, 64>(a, epi, stream);
    else launch_vec_tile<AT, BT, 16, 16, 128>(a, epi, stream);
}

// The VALU kernel for any NK-layout problem it can read; SFG_ERR_UNSUPPORTED
// for the QKV-RoPE epilogue and tiled weights.
int launch_vec(const GemmProblem& p, hipStream_t stream) {
    if (p.epilogue == kEpiQkvRope || p.b_layout != SFG_LAYOUT_NK) return SFG_ERR_UNSUPPORTED;
    VecArgs a{};
    a.a = p.a; a.lda = p.lda; a.a_rows = p.a_rows; a.a_rows_limit = p.a_rows ? p.a_rows_limit : p.m;
    a.b = p.b; a.ldb = p.ldb; a.scales = p.b_dtype == SFG_I8 ? p.b_scales : nullptr;
    a.b_group_stride = p.offsets ? p.b_group_stride : 0;
    a.s_group_stride = p.offsets ? p.s_group_stride : 0;
    a.c = p.c; a.c_dtype = p.c_dtype; a.ldc = p.ldc;
    a.residual = p.residual; a.ldr = p.ldr;
    a.m = p.m; a.n = p.n; a.k = p.k; a.offsets = p.offsets; a.groups = p.offsets ? p.groups : 1;
    if (p.a_dtype == SFG_F32 && p.b_dtype == SFG_F32) launch_vec_t<float, float>(a, p.epilogue, stream);
    else if (p.a_dtype == SFG_BF16 && p.b_dtype == SFG_BF16) launch_vec_t<uint16_t, uint16_t>(a, p.epilogue, stream);
    else if (p.a_dtype == SFG_BF16 && p.b_dtype == SFG_I8) launch_vec_t<uint16_t, int8_t>(a, p.epilogue, stream);
    else return SFG_ERR_UNSUPPORTED;
    return SFG_OK;
}

// ===========================================================================
// Host-side selection.
// ===========================================================================
namespace {

constexpr int kMaxWaves = 8;

// Waves per workgroup: enough that each wave owns at most one batch of chunks
// (4 at MT = 1, 2 otherwise) when K allows, capped so the LDS reduction
// buffer stays under 64 KB.
int skinny_waves(int64_t k, int mt, int nbt) {
    const int64_t chunks = k / kSkinnyChunk;
    const int64_t per_wave = mt == 1 ? kSkinnyBatch<1> : (mt == 2 ? kSkinnyBatch<2> : kSkinnyBatch<4>);
    int w = 4;
    while (w < kMaxWaves && chunks > per_wave * w) w *= 2;
    while (w > 4 && (w - 1) * mt * nbt * 1024 > 64 * 1024) w /= 2;
    return w;
}

template <int BDT, int MT, int NBT, int EPI>
void launch_skinny_w(const SkinnyArgs& a, dim3 grid, int waves, bool tiled, hipStream_t s) {
    if (tiled) {
        if (waves == 2) gemm_skinny_kernel<BDT, MT, NBT, EPI, 2, true><<<grid, 128, 0, s>>>(a);
        else if (waves == 4) gemm_skinny_kernel<BDT, MT, NBT, EPI, 4, true><<<grid, 256, 0, s>>>(a);
        else gemm_skinny_kernel<BDT, MT, NBT, EPI, 8, true><<<grid, 512, 0, s>>>(a);
    } else {
        if (waves == 2) gemm_skinny_kernel<BDT, MT, NBT, EPI, 2, false><<<grid, 128, 0, s>>>(a);
        else if (waves == 4) gemm_skinny_kernel<BDT, MT, NBT, EPI, 4, false><<<grid, 256, 0, s>>>(a);
        else gemm_skinny_kernel<BDT, MT, NBT, EPI, 8, false><<<grid, 512, 0, s>>>(a);
    }
}

template <int BDT, int MT>
void launch_skinny_e(const SkinnyArgs& a, dim3 grid, int nbt, int waves, int epi, bool tiled,
                     hipStream_t s) {
    switch (epi) {
        case SFG_EPI_NONE:
            if (nbt == 1) launch_skinny_w<BDT, MT, 1, SFG_EPI_NONE>(a, grid, waves, tiled, s);
            else launch_skinny_w<BDT, MT, 2, SFG_EPI_NONE>(a, grid, waves, tiled, s);
            break;
        case SFG_EPI_RESIDUAL:
            if (nbt == 1) launch_skinny_w<BDT, MT, 1, SFG_EPI_RESIDUAL>(a, grid, waves, tiled, s);
            else launch_skinny_w<BDT, MT, 2, SFG_EPI_RESIDUAL>(a, grid, waves, tiled, s);
            break;
        case SFG_EPI_SWIGLU: launch_skinny_w<BDT, MT, 2, SFG_EPI_SWIGLU>(a, grid, waves, tiled, s); break;
        default: launch_skinny_w<BDT, MT, 2, SFG_EPI_GLU_SILU_UP>(a, grid, waves, tiled, s); break;
    }
}

// Grouped problems: four B tiles (GLU: two gate + two up) per two-wave
// workgroup.
template <int BDT, int MT, int EPI>
void launch_skinny_g4(const SkinnyArgs& a, dim3 grid, bool tiled, hipStream_t s) {
    if (tiled) gemm_skinny_kernel<BDT, MT, 4, EPI, 2, true><<<grid, 128, 0, s>>>(a);
    else gemm_skinny_kernel<BDT, MT, 4, EPI, 2, false><<<grid, 128, 0, s>>>(a);
}
template <int BDT, int MT>
void launch_skinny_grouped4(const SkinnyArgs& a, dim3 grid, int epi, bool tiled, hipStream_t s) {
    switch (epi) {
        case SFG_EPI_NONE: launch_skinny_g4<BDT, MT, SFG_EPI_NONE>(a, grid, tiled, s); break;
        case SFG_EPI_RESIDUAL: launch_skinny_g4<BDT, MT, SFG_EPI_RESIDUAL>(a, grid, tiled, s); break;
        case SFG_EPI_SWIGLU: launch_skinny_g4<BDT, MT, SFG_EPI_SWIGLU>(a, grid, tiled, s); break;
        default: launch_skinny_g4<BDT, MT, SFG_EPI_GLU_SILU_UP>(a, grid, tiled, s); break;
    }
}

template <int BDT>
void launch_skinny_b(const SkinnyArgs& a, dim3 grid, int mt, int nbt, int waves, int epi,
                     bool tiled, hipStream_t s) {
    if (mt == 1) launch_skinny_e<BDT, 1>(a, grid, nbt, waves, epi, tiled, s);
    else if (mt == 2) launch_skinny_e<BDT, 2>(a, grid, nbt, waves, epi, tiled, s);
    else launch_skinny_e<BDT, 4>(a, grid, nbt, waves, epi, tiled, s);
}

template <int BDT>
void launch_big_b(const TiledArgs& a, dim3 grid, int tm, int tn, int epi, hipStream_t s) {
    switch (epi) {
        case SFG_EPI_NONE: gemm_mfma256_kernel<BDT, SFG_EPI_NONE><<<grid, 256, 0, s>>>(a, tm, tn); break;
        case SFG_EPI_RESIDUAL: gemm_mfma256_kernel<BDT, SFG_EPI_RESIDUAL><<<grid, 256, 0, s>>>(a, tm, tn); break;
        case SFG_EPI_SWIGLU: gemm_mfma256_kernel<BDT, SFG_EPI_SWIGLU><<<grid, 256, 0, s>>>(a, tm, tn); break;
        default: gemm_mfma256_kernel<BDT, SFG_EPI_GLU_SILU_UP><<<grid, 256, 0, s>>>(a, tm, tn); break;
    }
}

template <int BM, int BN, int NW = 4, bool PP = false, bool S64 = false>
void launch_dma_b(const TiledArgs& a, dim3 grid, int tm, int tn, int epi, hipStream_t s) {
    switch (epi) {
        case SFG_EPI_NONE: gemm_dma_kernel<BM, BN, NW, SFG_EPI_NONE, PP, S64><<<grid, NW * 64, 0, s>>>(a, tm, tn); break;
        case SFG_EPI_RESIDUAL: gemm_dma_kernel<BM, BN, NW, SFG_EPI_RESIDUAL, PP, S64><<<grid, NW * 64, 0, s>>>(a, tm, tn); break;
        case SFG_EPI_SWIGLU: gemm_dma_kernel<BM, BN, NW, SFG_EPI_SWIGLU, PP, S64><<<grid, NW * 64, 0, s>>>(a, tm, tn); break;
        case kEpiQkvRope: gemm_dma_kernel<BM, BN, NW, kEpiQkvRope, PP, S64><<<grid, NW * 64, 0, s>>>(a, tm, tn); break;
        default: gemm_dma_kernel<BM, BN, NW, SFG_EPI_GLU_SILU_UP, PP, S64><<<grid, NW * 64, 0, s>>>(a, tm, tn); break;
    }
}

// Output tile of the direct-to-LDS kernel.  SFG_TILE_AUTO: the largest tile
// (256 x 256 on the four-wave 64-k slab loop) that still gives at least 512
// workgroups (two per CU); smaller problems take smaller tiles.  A
// plan may name the tile instead (sfg_layer_desc::gemm_tile); results do not
// depend on it.
struct DmaShape { int bm, bn, waves; bool pingpong; bool slab64 = false; };
DmaShape dma_shape_of(int tile) {
    switch (tile) {
        case SFG_TILE_256x256_PP: return {256, 256, 8, true};
        case SFG_TILE_256x256_W8: return {256, 256, 8, false};
        case SFG_TILE_256x256_W4: return {256, 256, 4, false};
        case SFG_TILE_256x256_V: return {256, 256, 4, false, true};
        case SFG_TILE_256x128: return {256, 128, 4, false};
        case SFG_TILE_128x256: return {128, 256, 4, false};
        default: return {128, 128, 4, false};
    }
}
DmaShape pick_dma_shape(int64_t m, int64_t n_out, bool glu, int groups, int tile) {
    if (tile > SFG_TILE_AUTO && tile < SFG_TILE_COUNT) return dma_shape_of(tile);
    // Grouped products (expert W1|W3 and W2): the 256 x 256 tile once it has
    // work for half the CUs -- measured faster than 256 x 128 and 128 x 128 on
    // the MoE prefill shape although its tile count stays under 512.
    if (groups > 1 && ((m + 255) / 256 + groups) * ((n_out + (glu ? 127 : 255)) / (glu ? 128 : 256)) >= 128)
        return dma_shape_of(SFG_TILE_256x256_V);
    for (const int t : {SFG_TILE_256x256_V, SFG_TILE_256x128, SFG_TILE_128x128}) {
        const DmaShape sh = dma_shape_of(t);
        const int64_t cols = glu ? sh.bn / 2 : sh.bn;
        const int64_t tiles = ((m + sh.bm - 1) / sh.bm + (groups > 1 ? groups : 0)) * ((n_out + cols - 1) / cols);
        if (tiles >= 512) return sh;
    }
    return dma_shape_of(SFG_TILE_128x128);
}

template <int BDT>
void launch_tiled_b(const TiledArgs& a, dim3 grid, int epi, hipStream_t s) {
    switch (epi) {
        case SFG_EPI_NONE: gemm_mfma_kernel<BDT, SFG_EPI_NONE><<<grid, 256, 0, s>>>(a); break;
        case SFG_EPI_RESIDUAL: gemm_mfma_kernel<BDT, SFG_EPI_RESIDUAL><<<grid, 256, 0, s>>>(a); break;
        case SFG_EPI_SWIGLU: gemm_mfma_kernel<BDT, SFG_EPI_SWIGLU><<<grid, 256, 0, s>>>(a); break;
        default: gemm_mfma_kernel<BDT, SFG_EPI_GLU_SILU_UP><<<grid, 256, 0, s>>>(a); break;
    }
}

bool is_glu(int epi) { return epi == SFG_EPI_SWIGLU || epi == SFG_EPI_GLU_SILU_UP; }

// Skinny path handles at most this many rows per group per pass-set; dense
// problems above it, and grouped problems whose total rows exceed it, use the
// tiled kernel.
constexpr int64_t kSkinnyMaxRows = 64;
constexpr int64_t kSkinnyGroupedMaxTotal = 512;
// Problems with at least this many rows use the 256x128 kernel.
constexpr int64_t kBigMinRows = 1024;

// Partial-sum bytes of the split-K decode GEMM for m activation rows, nb B
// rows and reduction length k; 0 where the shape does not take it.
size_t splitk_bytes(int64_t m, int64_t nb, int64_t k) {
    if (m <= 32 || m > kSplitRows || k % kSplitKS != 0 || k / kSplitKS < 2 || nb % kSplitCols != 0) return 0;
    return static_cast<size_t>(k / kSplitKS) * m * nb * sizeof(float);
}

template <int BDT>
void launch_splitk_b(const SplitArgs& a, dim3 grid, bool tiled, hipStream_t s) {
    if (tiled) gemm_splitk_kernel<BDT, true><<<grid, 256, 0, s>>>(a);
    else gemm_splitk_kernel<BDT, false><<<grid, 256, 0, s>>>(a);
}

}  // namespace

bool gemm_qkv_rope_supported(const GemmProblem& p) {
    const QkvRopeOut& o = p.qkv;
    return p.a_dtype == SFG_BF16 && p.b_dtype == SFG_BF16 && !p.offsets && !p.a_rows &&
           p.b_layout == SFG_LAYOUT_NK && p.m >= kBigMinRows && p.k % kGK == 0 && o.rope && o.q &&
           o.k && o.vt && o.seq > 0 && o.seq % 4 == 0 && p.m % o.seq == 0 && o.q_heads > 0 &&
           o.kv_heads > 0 && p.n == (static_cast<int64_t>(o.q_heads) + 2 * o.kv_heads) * 128 &&
           o.ld_vt % 64 == 0 && o.ld_vt >= o.seq &&
           static_cast<uint64_t>(p.m) * p.lda * 2 <= 0xFFFFFFFFull &&
           static_cast<uint64_t>(p.n) * p.ldb * 2 <= 0xFFFFFFFFull;
}

int gemm_preferred_layout(int64_t rows, int64_t k, bool grouped) {
    const bool skinny = k % kSkinnyChunk == 0 &&
                        (grouped ? rows <= kSkinnyGroupedMaxTotal : rows <= kSkinnyMaxRows);
    return skinny ? SFG_LAYOUT_TILED : SFG_LAYOUT_NK;
}

size_t gemm_workspace_bytes(int64_t m, int64_t n, int64_t k) {
    return splitk_bytes(m, n, k);  // every other GEMM reduces inside its workgroup
}

int launch_gemm(const GemmProblem& problem, void* workspace, size_t workspace_bytes,
                hipStream_t stream) {
    GemmProblem p = problem;
    p.xcds = device_xcds(stream);
    const bool glu = is_glu(p.epilogue);
    if (p.epilogue == kEpiQkvRope && !gemm_qkv_rope_supported(p)) return SFG_ERR_UNSUPPORTED;
    if (p.a_dtype == SFG_F32) {
        if (p.b_dtype != SFG_F32) return SFG_ERR_UNSUPPORTED;
        return launch_vec(p, stream);
    }
    if (p.a_dtype != SFG_BF16 || (p.b_dtype != SFG_BF16 && p.b_dtype != SFG_I8))
        return SFG_ERR_UNSUPPORTED;
    if (p.b_dtype == SFG_I8 && p.b_scales == nullptr) return SFG_ERR_SHAPE;
    // every bf16 / int8 MFMA kernel reads A and B rows as 16-byte vectors and
    // steps k by 32: other rows and depths run on the VALU kernel
    const int64_t b_elem = p.b_dtype == SFG_I8 ? 1 : 2;
    if ((reinterpret_cast<uintptr_t>(p.a) & 15) || (reinterpret_cast<uintptr_t>(p.b) & 15) ||
        (p.lda * 2) % 16 != 0 || (p.ldb * b_elem) % 16 != 0 || p.k % kTK != 0)
        return launch_vec(p, stream);
    const int groups = p.offsets ? p.groups : 1;
    // 33..64 dense rows: split-K slices when the caller's workspace holds the
    // partial sums (sized by gemm_workspace_bytes).
    const int64_t nb = glu ? 2 * p.n : p.n;
    const size_t split_bytes =
        p.offsets || p.a_rows || p.epilogue == kEpiQkvRope ? 0 : splitk_bytes(p.m, nb, p.k);
    if (split_bytes > 0 && workspace && workspace_bytes >= split_bytes) {
        SplitArgs a{static_cast<const uint16_t*>(p.a), p.lda, p.b, p.ldb, static_cast<float*>(workspace),
                    p.m, nb, p.k};
        const dim3 grid(static_cast<unsigned>(nb / kSplitCols), static_cast<unsigned>(p.k / kSplitKS));
        const bool tiled = p.b_layout == SFG_LAYOUT_TILED;
        if (p.b_dtype == SFG_I8) launch_splitk_b<SFG_I8>(a, grid, tiled, stream);
        else launch_splitk_b<SFG_BF16>(a, grid, tiled, stream);
        SplitReduceArgs r{a.part, static_cast<int>(p.k / kSplitKS), p.b_scales, p.c, p.c_dtype, p.ldc,
                          p.residual, p.ldr, p.m, p.n, nb};
        const dim3 rgrid(static_cast<unsigned>((p.m * p.n / 4 + 255) / 256));
        switch (p.epilogue) {
            case SFG_EPI_NONE: gemm_splitk_reduce_kernel<SFG_EPI_NONE><<<rgrid, 256, 0, stream>>>(r); break;
            case SFG_EPI_RESIDUAL: gemm_splitk_reduce_kernel<SFG_EPI_RESIDUAL><<<rgrid, 256, 0, stream>>>(r); break;
            case SFG_EPI_SWIGLU: gemm_splitk_reduce_kernel<SFG_EPI_SWIGLU><<<rgrid, 256, 0, stream>>>(r); break;
            default: gemm_splitk_reduce_kernel<SFG_EPI_GLU_SILU_UP><<<rgrid, 256, 0, stream>>>(r); break;
        }
        return SFG_OK;
    }
    // The skinny kernel streams K in 128-element chunks and writes whole
    // 16-column tiles; other K, and an N its tiles do not divide, go to the
    // tiled or VALU kernels (which mask a ragged last column tile) when B is
    // [N][K].  Fragment-tiled B is read by the skinny kernel only.
    const bool skinny_rows = p.k % kSkinnyChunk == 0 &&
                             (p.offsets ? (p.m <= kSkinnyGroupedMaxTotal) : (p.m <= kSkinnyMaxRows));
    // grouped problems: 32 rows per pass covers the typical decode expert
    const int64_t rows_hint = p.offsets ? 32 : p.m;
    // grouped: four B tiles per workgroup (GLU: two gate + two up) halve
    // the activation re-reads per weight byte
    const bool g4 = p.offsets && p.n % (glu ? 32 : 64) == 0;
    int nbt = g4 ? 4 : (glu ? 2 : (rows_hint <= 16 ? 1 : 2));
    if (!glu && !g4 && p.n % (16 * nbt) != 0) nbt = 1;  // widths of an odd number of 16-column tiles
    const int64_t tile_cols = glu ? 16 * nbt / 2 : 16 * nbt;
    const bool skinny = skinny_rows && p.n % tile_cols == 0;
    if (skinny_rows && !skinny && p.b_layout == SFG_LAYOUT_TILED) return SFG_ERR_UNSUPPORTED;
    if (skinny) {
        const int mt = rows_hint <= 16 ? 1 : (rows_hint <= 32 ? 2 : 4);
        // A grouped launch already has groups x N/16 workgroups, several per
        // CU: two waves each keeps the K split (and its LDS reduction) short.
        // So does a 16-row GLU product up to K = 2048 (two load batches per
        // wave; measured faster than four waves on the decode gate|up).
        const bool two = p.offsets || (glu && mt == 1 && p.k <= 2048);
        const int waves = two ? 2 : skinny_waves(p.k, mt, nbt);
        SkinnyArgs a{};
        a.a = static_cast<const uint16_t*>(p.a); a.lda = p.lda; a.a_rows = p.a_rows;
        a.a_rows_limit = p.a_rows ? p.a_rows_limit : p.m;
        a.b = p.b; a.ldb = p.ldb; a.scales = p.b_scales;
        a.b_group_stride = p.b_group_stride; a.s_group_stride = p.s_group_stride;
        a.c = p.c; a.c_dtype = p.c_dtype; a.ldc = p.ldc;
        a.residual = p.residual; a.ldr = p.ldr;
        a.m = p.m; a.n = p.n; a.k = p.k; a.offsets = p.offsets;
        const dim3 grid(static_cast<unsigned>(p.n / tile_cols), 1u, static_cast<unsigned>(groups));
        const bool tiled = p.b_layout == SFG_LAYOUT_TILED;
        if (g4) {  // grouped problems always run 32 rows per pass (mt == 2)
            if (p.b_dtype == SFG_I8) launch_skinny_grouped4<SFG_I8, 2>(a, grid, p.epilogue, tiled, stream);
            else launch_skinny_grouped4<SFG_BF16, 2>(a, grid, p.epilogue, tiled, stream);
            return SFG_OK;
        }
        if (p.b_dtype == SFG_I8) launch_skinny_b<SFG_I8>(a, grid, mt, nbt, waves, p.epilogue, tiled, stream);
        else launch_skinny_b<SFG_BF16>(a, grid, mt, nbt, waves, p.epilogue, tiled, stream);
        return SFG_OK;
    }
    if (p.b_layout == SFG_LAYOUT_TILED) return SFG_ERR_UNSUPPORTED;  // tiled weights feed the skinny kernel only
    // The direct-to-LDS and 128 x 128 kernels mask a ragged last column tile;
    // the 256 x 128 register-staged kernel needs whole tiles.
    const bool whole_n = p.n % (glu ? 64 : 128) == 0;
    const bool big = p.k % kGK == 0 && p.m >= kBigMinRows;
    TiledArgs a{};
    a.a = static_cast<const uint16_t*>(p.a); a.lda = p.lda; a.a_rows = p.a_rows;
    a.a_rows_limit = p.a_rows ? p.a_rows_limit : p.m;
    a.b = p.b; a.ldb = p.ldb; a.scales = p.b_scales;
    a.b_group_stride = p.b_group_stride; a.s_group_stride = p.s_group_stride;
    a.c = p.c; a.c_dtype = p.c_dtype; a.ldc = p.ldc;
    a.residual = p.residual; a.ldr = p.ldr;
    a.m = p.m; a.n = p.n; a.k = p.k; a.offsets = p.offsets; a.groups = groups;
    a.qkv = p.qkv;
    a.xcds = p.xcds;
    // the direct-to-LDS kernel addresses each operand with 32-bit byte offsets;
    // a gathered zero row's loads sit at A's end plus the k offset
    const bool fits32 = static_cast<uint64_t>(a.a_rows_limit) * p.lda * 2 +
                                (p.a_rows ? static_cast<uint64_t>(p.k) * 2 + 64 : 0) <= 0xFFFFFFFFull &&
                        static_cast<uint64_t>(glu ? 2 : 1) * p.n * p.ldb * 2 <= 0xFFFFFFFFull;
    if (big && fits32 && p.b_dtype == SFG_BF16) {
        const DmaShape sh = pick_dma_shape(p.m, p.n, glu, groups, p.tile);
        const int64_t cols = glu ? sh.bn / 2 : sh.bn;
        const int64_t tn = (p.n + cols - 1) / cols;
        const int64_t tm = (p.m + sh.bm - 1) / sh.bm;
        const dim3 grid = p.offsets ? dim3(static_cast<unsigned>(tn), static_cast<unsigned>(tm + groups))
                                    : dim3(static_cast<unsigned>(tm * tn));
        const int itm = p.offsets ? 0 : static_cast<int>(tm);
        static_assert(kGK % 64 == 0, "the 256 x 256 V tile walks 64-k slabs");
        if (sh.slab64)
            launch_dma_b<256, 256, 4, false, true>(a, grid, itm, static_cast<int>(tn), p.epilogue, stream);
        else if (sh.bm == 256 && sh.bn == 256 && sh.pingpong)
            launch_dma_b<256, 256, 8, true>(a, grid, itm, static_cast<int>(tn), p.epilogue, stream);
        else if (sh.bm == 256 && sh.bn == 256 && sh.waves == 8) launch_dma_b<256, 256, 8>(a, grid, itm, static_cast<int>(tn), p.epilogue, stream);
        else if (sh.bm == 256 && sh.bn == 256) launch_dma_b<256, 256>(a, grid, itm, static_cast<int>(tn), p.epilogue, stream);
        else if (sh.bm == 256) launch_dma_b<256, 128>(a, grid, itm, static_cast<int>(tn), p.epilogue, stream);
        else if (sh.bn == 256) launch_dma_b<128, 256>(a, grid, itm, static_cast<int>(tn), p.epilogue, stream);
        else launch_dma_b<128, 128>(a, grid, itm, static_cast<int>(tn), p.epilogue, stream);
        return SFG_OK;
    }
    if (big && whole_n) {
        const int64_t tn = glu ? p.n / 64 : p.n / 128;
        if (p.offsets) {
            const dim3 grid(static_cast<unsigned>(tn), static_cast<unsigned>((p.m + kGM - 1) / kGM + groups));
            if (p.b_dtype == SFG_I8) launch_big_b<SFG_I8>(a, grid, 0, static_cast<int>(tn), p.epilogue, stream);
            else launch_big_b<SFG_BF16>(a, grid, 0, static_cast<int>(tn), p.epilogue, stream);
        } else {
            const int64_t tm = (p.m + kGM - 1) / kGM;
            const dim3 grid(static_cast<unsigned>(tm * tn));
            if (p.b_dtype == SFG_I8) launch_big_b<SFG_I8>(a, grid, static_cast<int>(tm), static_cast<int>(tn), p.epilogue, stream);
            else launch_big_b<SFG_BF16>(a, grid, static_cast<int>(tm), static_cast<int>(tn), p.epilogue, stream);
        }
        return SFG_OK;
    }
    const int64_t row_tiles = p.offsets ? (p.m + kTM - 1) / kTM + groups : (p.m + kTM - 1) / kTM;
    const dim3 grid(static_cast<unsigned>(glu ? (p.n + 63) / 64 : (p.n + 127) / 128), static_cast<unsigned>(row_tiles));
    if (p.b_dtype == SFG_I8) launch_tiled_b<SFG_I8>(a, grid, p.epilogue, stream);
    else launch_tiled_b<SFG_BF16>(a, grid, p.epilogue, stream);
    return SFG_OK;
}

}  // namespace sfg
