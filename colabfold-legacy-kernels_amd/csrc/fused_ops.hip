// LayerNorm-fused pair-stack projections for gfx950 (CDNA4): ln_gdp, trimul_epilogue,
// ln_projection, output_projection and transition.
//
// Semantics follow the reference (cuda/volta_ops.cu:330-641, cuda/volta_gdp.h, FFI validation in
// cuda/volta_fused_ffi.h:16-259): LayerNorm with two-pass fp32 statistics and its output rounded
// to fp16 before the GEMM; fp16 operands with fp32 accumulation; sigmoid gates; the transition's
// hidden activation rounded to fp16; keep decisions per row tile of 64 (32 for the tri-mul
// epilogue and the 256-channel transition), rows past M counting as `other`.
//
// Layout on the chip. Workgroups are persistent (a grid of about one per CU, each looping over
// row tiles), so a layer's weights are read from HBM once per workgroup and then stay in LDS.
// Every matrix in LDS is stored "fragment-major": for operand block b and contraction step ks,
// the 64 lanes' 16-byte MFMA operands are 64 consecutive chunks, so a wave's operand read is one
// conflict-free 1 KB sweep and no row padding is needed (which is what lets a 512 x 128 weight
// and a 64-row activation tile share one CU's 160 KB). Row-major results use the transposed
// product out^T = W X^T, whose accumulator gives a lane 8 consecutive columns of one row (a
// 16-byte store); channel-major results use out = X W^T, giving a lane 16 consecutive rows of
// one channel.
#include <type_traits>

#include "clk_common.h"

namespace clk {

constexpr int kFThreads = 256;
constexpr int kFWaves = kFThreads / kWave;
constexpr int kTileRows = 64;
constexpr int kProjThreads = 512;  // the projections' workgroup: 8 waves share the weights
constexpr int kEpiThreads = 1024;  // the tri-mul epilogue's workgroup: 16 waves share one copy of the weights
// ln_gdp: at K = 64 three 4-wave workgroups fit a CU (LDS and registers), at K = 128 one, which
// then runs 8 waves
template <int K>
constexpr int gdp_threads() { return K == 64 ? 256 : 512; }

enum TileWork { kCompute = 0, kPadding = 1, kSkip = 2 };

__device__ __forceinline__ half8 fzero8() {
    half8 z;
#pragma unroll
    for (int j = 0; j < 8; ++j) z[j] = (half_t)0.f;
    return z;
}
__device__ __forceinline__ half8 fld8(const half_t* p) { return *reinterpret_cast<const half8*>(p); }
__device__ __forceinline__ void fst8(half_t* p, half8 v) { *reinterpret_cast<half8*>(p) = v; }
// A streaming (nontemporal) 16-byte store, for outputs that no later kernel of the op reads back
// soon; measured faster for the wide outputs of ln_projection at c = 128 and ln_gdp, slower for
// ln_projection at c = 64, where two workgroups share a CU.
__device__ __forceinline__ void fst8_nt(half_t* p, half8 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<half8*>(p));
}

// operand chunk (block, step, lane) of a fragment-major matrix with KS contraction steps
__device__ __forceinline__ int frag(int block, int ks, int KS, int lane) {
    return ((block * KS + ks) * kWave + lane) * 8;
}

// A-operand row r of block b for a transposed product: blocks pair up so that the accumulator
// gives lane group g the 8 consecutive outputs 32 (b/2) + 8 g .. +7
__device__ __forceinline__ int pair_row(int b, int r) {
    return 32 * (b >> 1) + 8 * (r >> 2) + 4 * (b & 1) + (r & 3);
}

// A-operand row r of row block rb for a channel-major product: lane group g then holds the 16
// consecutive rows 16 g .. +15 across the four row blocks
__device__ __forceinline__ int quad_row(int rb, int r) { return 16 * (r >> 2) + 4 * rb + (r & 3); }

// What a row tile does, with the reference's rule (cuda/volta_gdp.h:114-136): compute when a
// keep is above zero, write padding when all are at most zero and one is zero, skip otherwise.
// Rows at or past M read as `other`. Every thread of the block must call it.
__device__ __forceinline__ int tile_work(const half_t* keep, int M, int m0, int R, float other) {
    if (keep == nullptr) return kCompute;
    bool live = false, zero = false;
    for (int r = threadIdx.x; r < R; r += blockDim.x) {
        const float k = m0 + r < M ? (float)keep[m0 + r] : other;
        live |= k > 0.f;
        zero |= k == 0.f;
    }
    if (__syncthreads_or(live)) return kCompute;
    return __syncthreads_or(zero) ? kPadding : kSkip;
}

// Weight rows [0, rows) of a row-major [rows][K] fp16 matrix into fragment-major LDS, nblocks
// blocks of 16 rows; PAIRED uses pair_row, otherwise block b holds rows 16 b .. +15. Rows past
// `rows` are zero.
template <int K, bool PAIRED>
__device__ __forceinline__ void load_weight_frags(half_t* dst, const half_t* W, int rows, int nblocks,
                                                  int row0 = 0) {
    constexpr int KS = K / 32;
    for (int i = threadIdx.x; i < nblocks * KS * kWave; i += blockDim.x) {
        const int lane = i % kWave, t = i / kWave, ks = t % KS, b = t / KS;
        const int r = PAIRED ? pair_row(b, lane & 15) : 16 * b + (lane & 15);
        const int col = 32 * ks + 8 * (lane >> 4);
        fst8(dst + i * 8, r < rows ? fld8(W + (int64_t)(row0 + r) * K + col) : fzero8());
    }
}

// ---- LayerNorm of a row tile into fragment-major LDS ---------------------------------------
//
// R rows of a row-major [M][K] fp16 matrix; 256 / R threads per row, each holding K / (8 TPR)
// 16-byte chunks (chunk c = part + TPR j). QUAD picks the channel-major A-operand layout
// (quad_row), otherwise the transposed product's B-operand layout.
template <int K, int R, int TH = kFThreads>
struct RowTile {
    static constexpr int kTPR = TH / R;
    static_assert(K / 8 >= kTPR, "each thread holds at least one 16-byte chunk of its row");
    static constexpr int kChunks = K / 8 / kTPR;
    half8 v[kChunks];
};

template <int K, int R, int TH>
__device__ __forceinline__ void fetch_rows(RowTile<K, R, TH>& t, const half_t* x, int M, int m0) {
    constexpr int TPR = RowTile<K, R, TH>::kTPR;
    const int row = threadIdx.x / TPR, part = threadIdx.x % TPR;
#pragma unroll
    for (int j = 0; j < RowTile<K, R, TH>::kChunks; ++j) {
        const int c = part + TPR * j;
        t.v[j] = m0 + row < M ? fld8(x + (int64_t)(m0 + row) * K + 8 * c) : fzero8();
    }
}

template <int TPR>
__device__ __forceinline__ float group_sum(float s) {
    if (TPR >= 2) s += __shfl_xor(s, 1);
    if (TPR >= 4) s += __shfl_xor(s, 2);
    if (TPR >= 8) s += __shfl_xor(s, 4);
    return s;
}

template <int K, int R, bool QUAD, bool LN, int TH, bool BF = false>
__device__ __forceinline__ void ln_rows_to_frags(half_t* Xf, const RowTile<K, R, TH>& t,
                                                 const float* sc, const float* of, float eps) {
    using RT = RowTile<K, R, TH>;
    constexpr int TPR = RT::kTPR, KS = K / 32;
    const int row = threadIdx.x / TPR, part = threadIdx.x % TPR;
    float mean = 0.f, rstd = 1.f;
    if constexpr (LN) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < RT::kChunks; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) s += act_get<BF>(t.v[j], e);
        mean = group_sum<TPR>(s) * (1.f / K);
        float q = 0.f;
#pragma unroll
        for (int j = 0; j < RT::kChunks; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = act_get<BF>(t.v[j], e) - mean;
                q += d * d;
            }
        rstd = __builtin_amdgcn_rsqf(group_sum<TPR>(q) * (1.f / K) + eps);
    }
    int rb, rl;
    if (QUAD) {
        rb = (row >> 2) & 3;
        rl = 4 * (row >> 4) + (row & 3);
        rb += 4 * (row / 64);  // tiles taller than 64 rows stack 4-block groups
        rl = 4 * ((row & 63) >> 4) + (row & 3);
    } else {
        rb = row >> 4;
        rl = row & 15;
    }
#pragma unroll
    for (int j = 0; j < RT::kChunks; ++j) {
        const int c = part + TPR * j;
        half8 y;
        if constexpr (LN) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int col = 8 * c + e;
                y[e] = (half_t)((act_get<BF>(t.v[j], e) - mean) * rstd * sc[col] + of[col]);
            }
        } else if constexpr (BF) {
            // bf16 to fp16: exact within fp16's normal range
#pragma unroll
            for (int e = 0; e < 8; ++e) y[e] = (half_t)act_get<true>(t.v[j], e);
        } else {
            y = t.v[j];
        }
        fst8(Xf + frag(rb, c >> 2, KS, rl + 16 * (c & 3)), y);
    }
}

// ---- ln_projection / output_projection --------------------------------------------------

struct ProjArgs {
    const half_t* x;
    const float* scale;
    const float* offset;
    const half_t* wT;        // [n][K]
    const half_t* wbT;       // [heads][K]
    const half_t* b;         // [n] or null
    const half_t* residual;  // [M][n] or null (may alias out)
    const half_t* keep;      // [M] or null
    half_t* out;             // [M][n]
    half_t* bias;            // [heads][M]
    int M, n, heads;
    int cols;                // columns per workgroup column chunk (multiple of 32)
    float eps;
};

// TH threads share the LDS-resident weights. The 64 x ncols output tile is split into items of
// one column pair (32 outputs) and 4 / split row blocks: with at least as many pairs as waves a
// wave takes whole pairs, otherwise `split` waves share a pair and divide its four row blocks.
template <int K, bool LN, int TH, bool BF>
__global__ __launch_bounds__(TH) void proj_kernel(ProjArgs a) {
    constexpr int KS = K / 32, TW = TH / kWave;
    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    const int col0 = blockIdx.y * a.cols;
    const int ncols = min(a.cols, a.n - col0);
    const bool do_heads = blockIdx.y == 0 && a.heads > 0;
    const int npairs = ncols > 0 ? ncols / 32 : 0;
    half_t* Wf = lds;                                  // npairs * 2 blocks
    half_t* Hf = Wf + npairs * 32 * K;                 // one block of head rows
    half_t* Xf = Hf + (do_heads ? 16 * K : 0);         // 4 row blocks
    float* sc = reinterpret_cast<float*>(Xf + kTileRows * K);
    float* of = sc + K;

    if (npairs > 0) load_weight_frags<K, true>(Wf, a.wT, ncols, 2 * npairs, col0);
    if (do_heads) load_weight_frags<K, false>(Hf, a.wbT, a.heads, 1);
    if constexpr (LN) {
        for (int i = threadIdx.x; i < K; i += TH) {
            sc[i] = a.scale[i];
            of[i] = a.offset[i];
        }
    }

    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int r16 = lane & 15, g = lane >> 4;
    const int tiles = (a.M + kTileRows - 1) / kTileRows;
    const int split = npairs >= TW || npairs == 0 ? 1 : min(4, TW / npairs);
    const int rbn = 4 / split, rb0 = (wave % split) * rbn;
    const int pair0 = wave / split, pstride = TW / split;
    const bool heads_wave = do_heads && wave == TW - 1;

    RowTile<K, kTileRows, TH> xt;
    if (blockIdx.x < tiles) fetch_rows<K, kTileRows>(xt, a.x, a.M, blockIdx.x * kTileRows);
    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
        const int m0 = tile * kTileRows;
        const int work = tile_work(a.keep, a.M, m0, kTileRows, -1.f);
        if (work != kCompute) {
            if (work == kPadding) {
                // with a residual the output aliases it, which padding keeps
                if (ncols > 0 && a.residual == nullptr) {
                    for (int i = threadIdx.x; i < kTileRows * ncols / 8; i += TH) {
                        const int r = i / (ncols / 8), c = (i % (ncols / 8)) * 8;
                        if (m0 + r < a.M) fst8(a.out + (int64_t)(m0 + r) * a.n + col0 + c, fzero8());
                    }
                }
                if (do_heads) {
                    for (int i = threadIdx.x; i < kTileRows * a.heads; i += TH) {
                        const int h = i / kTileRows, r = i % kTileRows;
                        if (m0 + r < a.M) a.bias[(int64_t)h * a.M + m0 + r] = (half_t)0.f;
                    }
                }
            }
            if (tile + gridDim.x < tiles) fetch_rows<K, kTileRows>(xt, a.x, a.M, (tile + gridDim.x) * kTileRows);
            continue;
        }
        __syncthreads();  // the previous tile's operand reads are done
        ln_rows_to_frags<K, kTileRows, false, LN, TH, BF>(Xf, xt, sc, of, a.eps);
        __syncthreads();
        if (tile + gridDim.x < tiles) fetch_rows<K, kTileRows>(xt, a.x, a.M, (tile + gridDim.x) * kTileRows);

        half8 xop[4][KS];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                if (rb >= rb0 && rb < rb0 + rbn) xop[rb][ks] = fld8(Xf + frag(rb, ks, KS, lane));
            }

        for (int cp = pair0; cp < npairs; cp += pstride) {
            float4v acc[2][4];
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) acc[hb][rb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) {
                    const half8 w = fld8(Wf + frag(2 * cp + hb, ks, KS, lane));
#pragma unroll
                    for (int rb = 0; rb < 4; ++rb) {
                        if (rb >= rb0 && rb < rb0 + rbn) acc[hb][rb] = mfma16x16x32(w, xop[rb][ks], acc[hb][rb]);
                    }
                }
            }
            const int col = col0 + 32 * cp + 8 * g;
            float bv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) bv[j] = 0.f;
            if constexpr (!LN) {
                const half8 b8 = fld8(a.b + col);
#pragma unroll
                for (int j = 0; j < 8; ++j) bv[j] = (float)b8[j];
            }
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const int row = m0 + 16 * rb + r16;
                if (rb < rb0 || rb >= rb0 + rbn || row >= a.M) continue;
                half_t* dst = a.out + (int64_t)row * a.n + col;
                half8 o;
                if constexpr (LN) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] = act_cvt<BF>(acc[j >> 2][rb][j & 3]);
                } else if (a.residual != nullptr) {
                    const half8 res = fld8(a.residual + (int64_t)row * a.n + col);
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] = act_cvt<BF>(acc[j >> 2][rb][j & 3] + bv[j] + act_get<BF>(res, j));
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] = act_cvt<BF>(acc[j >> 2][rb][j & 3] + bv[j]);
                }
                fst8(dst, o);
            }
        }
        if (heads_wave) {
            // the head-bias block reads every row block
            half8 hx[4][KS];
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) hx[rb][ks] = fld8(Xf + frag(rb, ks, KS, lane));
            float4v acc[4];
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) acc[rb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const half8 w = fld8(Hf + frag(0, ks, KS, lane));
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) acc[rb] = mfma16x16x32(w, hx[rb][ks], acc[rb]);
            }
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const int row = m0 + 16 * rb + r16;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int h = 4 * g + i;
                    if (h < a.heads && row < a.M) a.bias[(int64_t)h * a.M + row] = act_cvt<BF>(acc[rb][i]);
                }
            }
        }
    }
}

// The same projection with a fixed shape of work, for the common case: no keep mask, and every
// wave owning exactly PAIRS column pairs (all four row blocks). Each wave then issues a fixed
// number of stores per tile, and the next tile's rows are prefetched unconditionally (clamped to
// the last tile), so the loop over whole tiles is straight-line: the wait for the prefetched rows
// covers only them, not the stores issued after them. The partial last tile, if any, follows the
// loop with per-row checks.
// At K = 64 two workgroups share a CU (LDS allows it), so the kernel is held to 128 VGPRs.
template <int K, bool LN, int TH, int PAIRS, bool BF>
__global__ __launch_bounds__(TH, K == 64 ? 4 : 1) void proj_fast_kernel(ProjArgs a) {
    constexpr int KS = K / 32, TW = TH / kWave, NP = PAIRS * TW;
    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    const int col0 = blockIdx.y * a.cols;
    const bool do_heads = blockIdx.y == 0 && a.heads > 0;
    half_t* Wf = lds;                           // NP * 2 blocks
    half_t* Hf = Wf + NP * 32 * K;              // one block of head rows
    half_t* Xf = Hf + (do_heads ? 16 * K : 0);  // 4 row blocks
    float* sc = reinterpret_cast<float*>(Xf + kTileRows * K);
    float* of = sc + K;

    load_weight_frags<K, true>(Wf, a.wT, NP * 32, 2 * NP, col0);
    if (do_heads) load_weight_frags<K, false>(Hf, a.wbT, a.heads, 1);
    if constexpr (LN) {
        for (int i = threadIdx.x; i < K; i += TH) {
            sc[i] = a.scale[i];
            of[i] = a.offset[i];
        }
    }

    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int r16 = lane & 15, g = lane >> 4;
    const int tiles = (a.M + kTileRows - 1) / kTileRows, full = a.M / kTileRows;
    const bool heads_wave = do_heads && wave == TW - 1;

    // the output projection's bias of this lane's columns, the same for every tile
    float bv[PAIRS][8];
#pragma unroll
    for (int pp = 0; pp < PAIRS; ++pp) {
        const int col = col0 + 32 * (wave + pp * TW) + 8 * g;
        half8 b8 = fzero8();
        if constexpr (!LN) b8 = fld8(a.b + col);
#pragma unroll
        for (int j = 0; j < 8; ++j) bv[pp][j] = (float)b8[j];
    }

    // rows of tile t (rows past M repeat the last row; their outputs are never stored)
    RowTile<K, kTileRows, TH> xt;
    const auto fetch = [&](int t) {
        constexpr int TPR = RowTile<K, kTileRows, TH>::kTPR;
        const int row = threadIdx.x / TPR, part = threadIdx.x % TPR;
        const int m = min(t * kTileRows + row, a.M - 1);
#pragma unroll
        for (int j = 0; j < RowTile<K, kTileRows, TH>::kChunks; ++j)
            xt.v[j] = fld8(a.x + (int64_t)m * K + 8 * (part + TPR * j));
    };

    const auto body = [&](int tile, auto full_tag) {
        constexpr bool kFull = decltype(full_tag)::value;
        const int m0 = tile * kTileRows;
        // this tile's residual, loaded before the next tile's rows so that waiting for it does
        // not wait for them
        half8 res[PAIRS][4];
        if (!LN && a.residual != nullptr) {
#pragma unroll
            for (int pp = 0; pp < PAIRS; ++pp)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    const int row = min(m0 + 16 * rb + r16, a.M - 1);
                    res[pp][rb] = fld8(a.residual + (int64_t)row * a.n + col0 + 32 * (wave + pp * TW) + 8 * g);
                }
        }
        __syncthreads();  // the previous tile's operand reads are done
        ln_rows_to_frags<K, kTileRows, false, LN, TH, BF>(Xf, xt, sc, of, a.eps);
        __syncthreads();
        fetch(min(tile + (int)gridDim.x, tiles - 1));

        half8 xop[4][KS];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) xop[rb][ks] = fld8(Xf + frag(rb, ks, KS, lane));

#pragma unroll
        for (int pp = 0; pp < PAIRS; ++pp) {
            const int cp = wave + pp * TW;
            float4v acc[2][4];
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) acc[hb][rb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) {
                    const half8 w = fld8(Wf + frag(2 * cp + hb, ks, KS, lane));
#pragma unroll
                    for (int rb = 0; rb < 4; ++rb) acc[hb][rb] = mfma16x16x32(w, xop[rb][ks], acc[hb][rb]);
                }
            }
            const int col = col0 + 32 * cp + 8 * g;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const int row = m0 + 16 * rb + r16;
                if (!kFull && row >= a.M) continue;
                half8 o;
                if constexpr (LN) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] = act_cvt<BF>(acc[j >> 2][rb][j & 3]);
                } else if (a.residual != nullptr) {
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        o[j] = act_cvt<BF>(acc[j >> 2][rb][j & 3] + bv[pp][j] + act_get<BF>(res[pp][rb], j));
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] = act_cvt<BF>(acc[j >> 2][rb][j & 3] + bv[pp][j]);
                }
                if constexpr (K == 128) {
                    fst8_nt(a.out + (int64_t)row * a.n + col, o);
                } else {
                    fst8(a.out + (int64_t)row * a.n + col, o);
                }
            }
        }
        if (heads_wave) {
            // the head-bias block reads every row block
            float4v acc[4];
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) acc[rb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const half8 w = fld8(Hf + frag(0, ks, KS, lane));
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) acc[rb] = mfma16x16x32(w, xop[rb][ks], acc[rb]);
            }
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const int row = m0 + 16 * rb + r16;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int h = 4 * g + i;
                    if (h < a.heads && (kFull || row < a.M)) a.bias[(int64_t)h * a.M + row] = act_cvt<BF>(acc[rb][i]);
                }
            }
        }
    };

    int tile = blockIdx.x;
    if constexpr (K == 128) {
        // the first whole tile runs before the loop, and the loop is reachable only through it, so
        // the loop is entered, like every later iteration, with a tile's stores issued after the
        // rows it prefetched: the wait at the top of a tile covers the rows and not the stores
        if (tile < full) {
            fetch(tile);
            body(tile, std::true_type{});
            for (tile += gridDim.x; tile < full; tile += gridDim.x) body(tile, std::true_type{});
        } else if (tile < tiles) {
            fetch(tile);
        }
    } else {
        // here a path reaches the loop straight from the fetch, so each tile starts by waiting for
        // the previous tile's stores as well: with two workgroups per CU and the write stream at
        // its limit, that measured 4% faster than leaving them in flight
        if (tile < tiles) fetch(tile);
        if (tile < full) {
            body(tile, std::true_type{});
            tile += gridDim.x;
        }
        for (; tile < full; tile += gridDim.x) body(tile, std::true_type{});
    }
    if (tile < tiles) body(tile, std::false_type{});
}

// The output projection (no LayerNorm, no head rows) as straight-line code, like the tri-mul
// epilogue: eight waves, wave w owning column pair w / SPLIT and RBW of the four row blocks; the
// next tile's keep values, rows and residual fetched before this tile's stores and consumed in the
// same iteration after them; the keep decision from a ballot of the tile's 64 rows; dropped
// buffer stores for skipped tiles, for padding that must keep the residual the output aliases,
// and for rows past M.
template <int K, int N, bool RES, bool BF>
__global__ __launch_bounds__(kProjThreads, 4) void outproj_kernel(ProjArgs a) {
    constexpr int TH = kProjThreads, KS = K / 32, TW = TH / kWave;
    constexpr int NPAIRS = N / 32, SPLIT = TW / NPAIRS, RBW = 4 / SPLIT;
    static_assert(TW % NPAIRS == 0 && 4 % SPLIT == 0, "whole row blocks per wave");
    constexpr uint32_t kDrop = 0x80000000u;  // a store offset past every tile's end
    using u32x4 = unsigned int __attribute__((ext_vector_type(4)));
    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    half_t* Wf = lds;           // N / 16 paired blocks
    half_t* Xf = Wf + N * K;    // 4 row blocks
    load_weight_frags<K, true>(Wf, a.wT, N, N / 16);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int r16 = lane & 15, g = lane >> 4;
    const int cp = wave / SPLIT, rb0 = (wave % SPLIT) * RBW;
    const int col = 32 * cp + 8 * g;
    const int tiles = (a.M + kTileRows - 1) / kTileRows;
    const int G = gridDim.x;
    const bool has_keep = a.keep != nullptr;
    // without a keep the descriptor has no bytes, and its loads return zeros without touching memory
    const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.keep), 0,
                                                     has_keep ? (uint32_t)a.M * 2u : 0u, 0x00020000);
    float bv[8];
    {
        const half8 b8 = fld8(a.b + col);
#pragma unroll
        for (int j = 0; j < 8; ++j) bv[j] = (float)b8[j];
    }

    // tile t's keep value of row m0 + lane, rows and residual (rows past M repeat row M - 1;
    // their results are dropped)
    unsigned short kraw;
    RowTile<K, kTileRows, TH> xt;
    half8 rs[RBW];
    const auto fetch = [&](int t) {
        const int m0 = t * kTileRows;
        kraw = __builtin_amdgcn_raw_buffer_load_b16(rk, (uint32_t)min(m0 + lane, a.M - 1) * 2u, 0, 0);
        constexpr int TPR = RowTile<K, kTileRows, TH>::kTPR;
        const int row = threadIdx.x / TPR, part = threadIdx.x % TPR;
        const int mx = min(m0 + row, a.M - 1);
#pragma unroll
        for (int j = 0; j < RowTile<K, kTileRows, TH>::kChunks; ++j)
            xt.v[j] = fld8(a.x + (int64_t)mx * K + 8 * (part + TPR * j));
        if constexpr (RES) {
#pragma unroll
            for (int i = 0; i < RBW; ++i)
                rs[i] = fld8(a.residual + (int64_t)min(m0 + 16 * (rb0 + i) + r16, a.M - 1) * N + col);
        }
    };
    // the reference's keep rule for the tile (rows past M count as -1, volta_gdp.h:114-136)
    int work = kCompute;
    float resf[RBW][8];
    const auto prepare = [&](int t) {
        const int m0 = t * kTileRows;
        const float k = m0 + lane < a.M ? (has_keep ? (float)__builtin_bit_cast(half_t, kraw) : 1.f) : -1.f;
        const uint64_t live = __ballot(k > 0.f), zero = __ballot(k == 0.f);
        work = live ? (int)kCompute : zero ? (int)kPadding : (int)kSkip;
        __syncthreads();  // the previous tile's operand reads are done
        ln_rows_to_frags<K, kTileRows, false, false, TH, BF>(Xf, xt, nullptr, nullptr, 0.f);
#pragma unroll
        for (int i = 0; i < RBW; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) resf[i][j] = RES ? pin_f32(act_get<BF>(rs[i], j)) : 0.f;  // here, not after the next fetch
        __syncthreads();
    };
    const auto gemm_store = [&](int t) {
        const int m0 = t * kTileRows;
        float4v acc[2][RBW];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int i = 0; i < RBW; ++i) acc[hb][i] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            half8 xop[RBW];
#pragma unroll
            for (int i = 0; i < RBW; ++i) xop[i] = fld8(Xf + frag(rb0 + i, ks, KS, lane));
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                const half8 w = fld8(Wf + frag(2 * cp + hb, ks, KS, lane));
#pragma unroll
                for (int i = 0; i < RBW; ++i) acc[hb][i] = mfma16x16x32(w, xop[i], acc[hb][i]);
            }
        }
        // the tile's rows as one buffer: rows past M lie past its end
        const uint32_t rows = (uint32_t)min(kTileRows, a.M - m0);
        const auto ro = __builtin_amdgcn_make_buffer_rsrc(a.out + (int64_t)m0 * N, 0, rows * N * 2u, 0x00020000);
        // with a residual the output aliases it, which padding keeps
        const bool store = work == kCompute || (!RES && work == kPadding);
#pragma unroll
        for (int i = 0; i < RBW; ++i) {
            half8 o;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                o[j] = act_cvt<BF>(work == kPadding ? 0.f : acc[j >> 2][i][j & 3] + bv[j] + resf[i][j]);
            const uint32_t off = (uint32_t)((16 * (rb0 + i) + r16) * N + col) * 2u;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), ro, store ? off : kDrop, 0, 0);
        }
    };

    int t = blockIdx.x;
    if (t >= tiles) return;
    fetch(t);
    prepare(t);
    for (;;) {
        const int nt = t + G;
        // the output may alias the residual: the next tile's rows are not this tile's
        fetch(min(nt, tiles - 1));
        gemm_store(t);
        if (nt >= tiles) break;
        t = nt;
        prepare(t);
    }
}

// ln_projection without a keep mask for n in {256, 512}: every store writes whole output rows.
// Each wave keeps the A operands of its PAIRS column pairs (W^T rows, in pair order) in registers,
// which leaves LDS free for the 64 x n output tile. A tile's products go to that tile in LDS
// (16-byte chunk c of row r at chunk c ^ (r % 16), so a wave's writes cover all banks), and after a
// barrier each wave stores whole rows: one 16-byte chunk per lane, so a store instruction writes
// one or two contiguous rows (1 KB). The loop is rotated like the other straight-line kernels:
// the next tile's rows are fetched before this tile's products and stores and normalised after
// them. The head-bias block (channel-major) is computed and stored by the last wave as before.
template <int K, int N, bool BF>
__global__ __launch_bounds__(kProjThreads, K == 64 ? 4 : 2) void proj_rows_kernel(ProjArgs a) {
    constexpr int TH = kProjThreads, KS = K / 32, TW = TH / kWave, PAIRS = N / 32 / TW;
    constexpr int RCH = N / 8;                   // 16-byte chunks of an output row
    constexpr int RPI = kWave / RCH;             // rows per store instruction
    constexpr int SPW = kTileRows / (TW * RPI);  // store instructions per wave and tile
    static_assert(PAIRS >= 1 && N % (32 * TW) == 0 && kWave % RCH == 0, "whole pairs and rows");
    using u32x4 = unsigned int __attribute__((ext_vector_type(4)));
    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    half_t* Ot = lds;                    // [64][N], swizzled chunks
    half_t* Xf = Ot + kTileRows * N;     // 4 row blocks
    half_t* Hf = Xf + kTileRows * K;     // one block of head rows
    float* sc = reinterpret_cast<float*>(Hf + 16 * K);
    float* of = sc + K;
    const bool do_heads = a.heads > 0;
    if (do_heads) load_weight_frags<K, false>(Hf, a.wbT, a.heads, 1);
    for (int i = threadIdx.x; i < K; i += TH) {
        sc[i] = a.scale[i];
        of[i] = a.offset[i];
    }
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int r16 = lane & 15, g = lane >> 4;
    const int tiles = (a.M + kTileRows - 1) / kTileRows;
    const int G = gridDim.x;
    const bool heads_wave = do_heads && wave == TW - 1;

    // A row r of block hb of pair cp = wave + TW pp is output column 32 cp + 8 (r / 4) + 4 hb + r % 4
    half8 wa[PAIRS][2][KS];
#pragma unroll
    for (int pp = 0; pp < PAIRS; ++pp)
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const int col = 32 * (wave + pp * TW) + 8 * (r16 >> 2) + 4 * hb + (r16 & 3);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) wa[pp][hb][ks] = fld8(a.wT + (int64_t)col * K + 32 * ks + 8 * g);
        }

    // rows of tile t (rows past M repeat row M - 1; their results are dropped)
    RowTile<K, kTileRows, TH> xt;
    const auto fetch = [&](int t) {
        constexpr int TPR = RowTile<K, kTileRows, TH>::kTPR;
        const int row = threadIdx.x / TPR, part = threadIdx.x % TPR;
        const int m = min(t * kTileRows + row, a.M - 1);
#pragma unroll
        for (int j = 0; j < RowTile<K, kTileRows, TH>::kChunks; ++j)
            xt.v[j] = fld8(a.x + (int64_t)m * K + 8 * (part + TPR * j));
    };
    const auto prepare = [&]() {
        __syncthreads();  // the previous tile's operand reads and output-tile reads are done
        ln_rows_to_frags<K, kTileRows, false, true, TH, BF>(Xf, xt, sc, of, a.eps);
        __syncthreads();
    };
    const auto compute_store = [&](int t) {
        const int m0 = t * kTileRows;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            half8 xop[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) xop[ks] = fld8(Xf + frag(rb, ks, KS, lane));
            const int row = 16 * rb + r16;
#pragma unroll
            for (int pp = 0; pp < PAIRS; ++pp) {
                float4v acc[2] = {float4v{0.f, 0.f, 0.f, 0.f}, float4v{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int hb = 0; hb < 2; ++hb) acc[hb] = mfma16x16x32(wa[pp][hb][ks], xop[ks], acc[hb]);
                half8 o;
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = act_cvt<BF>(acc[j >> 2][j & 3]);
                const int chunk = 4 * (wave + pp * TW) + g;
                fst8(Ot + row * N + 8 * (chunk ^ (row & 15)), o);
            }
            if (heads_wave) {
                float4v hacc = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) hacc = mfma16x16x32(fld8(Hf + frag(0, ks, KS, lane)), xop[ks], hacc);
                const int m = m0 + row;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int h = 4 * g + i;
                    if (h < a.heads && m < a.M) a.bias[(int64_t)h * a.M + m] = act_cvt<BF>(hacc[i]);
                }
            }
        }
        __syncthreads();  // the output tile is complete
        // the tile's rows as one buffer: rows past M lie past its end
        const uint32_t rows = (uint32_t)min(kTileRows, a.M - m0);
        const auto ro = __builtin_amdgcn_make_buffer_rsrc(a.out + (int64_t)m0 * N, 0, rows * N * 2u, 0x00020000);
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int row = (i * TW + wave) * RPI + lane / RCH, chunk = lane % RCH;
            const half8 v = fld8(Ot + row * N + 8 * (chunk ^ (row & 15)));
            const uint32_t off = (uint32_t)(row * N + 8 * chunk) * 2u;
            if constexpr (K == 128) {  // nontemporal, as measured for the wide output at c = 128
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), ro, off, 0, 2);
            } else {
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), ro, off, 0, 0);
            }
        }
    };

    int t = blockIdx.x;
    if (t >= tiles) return;
    fetch(t);
    prepare();
    for (;;) {
        const int nt = t + G;
        fetch(min(nt, tiles - 1));
        compute_store(t);
        if (nt >= tiles) break;
        t = nt;
        prepare();
    }
}

// ---- ln_gated_dual_proj ---------------------------------------------------------------------

struct LnGdpArgs {
    const half_t* x;
    const float* scale;
    const float* offset;
    const half_t *wpT, *bp, *wgT, *bg, *mask;
    half_t *left, *right;
    int M, P;
    float eps;
};

template <int K, int TH, bool BF>
__global__ __launch_bounds__(TH) void ln_gdp_kernel(LnGdpArgs a) {
    constexpr int KS = K / 32, TW = TH / kWave;
    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    const int nb = a.P / 16;
    half_t* Wp = lds;
    half_t* Wg = Wp + a.P * K;
    half_t* Xf = Wg + a.P * K;
    float* sc = reinterpret_cast<float*>(Xf + kTileRows * K);
    float* of = sc + K;
    load_weight_frags<K, false>(Wp, a.wpT, a.P, nb);
    load_weight_frags<K, false>(Wg, a.wgT, a.P, nb);
    for (int i = threadIdx.x; i < K; i += TH) {
        sc[i] = a.scale[i];
        of[i] = a.offset[i];
    }
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int r16 = lane & 15, g = lane >> 4;
    const int tiles = (a.M + kTileRows - 1) / kTileRows;
    const int ci = a.P / 2;
    const bool vec = (a.M & 7) == 0;

    RowTile<K, kTileRows, TH> xt;
    if (blockIdx.x < tiles) fetch_rows<K, kTileRows>(xt, a.x, a.M, blockIdx.x * kTileRows);
    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
        const int m0 = tile * kTileRows;
        // the mask is the keep: rows past M count as zero (volta_ops.cu:349)
        const int work = tile_work(a.mask, a.M, m0, kTileRows, 0.f);
        if (work != kCompute) {
            if (work == kPadding) {
                for (int i = threadIdx.x; i < kTileRows * ci; i += TH) {
                    const int c = i / kTileRows, r = i % kTileRows;
                    if (m0 + r < a.M) {
                        a.left[(int64_t)c * a.M + m0 + r] = (half_t)0.f;
                        a.right[(int64_t)c * a.M + m0 + r] = (half_t)0.f;
                    }
                }
            }
            if (tile + gridDim.x < tiles) fetch_rows<K, kTileRows>(xt, a.x, a.M, (tile + gridDim.x) * kTileRows);
            continue;
        }
        __syncthreads();
        ln_rows_to_frags<K, kTileRows, true, true, TH, BF>(Xf, xt, sc, of, a.eps);
        __syncthreads();
        if (tile + gridDim.x < tiles) fetch_rows<K, kTileRows>(xt, a.x, a.M, (tile + gridDim.x) * kTileRows);

        half8 xop[4][KS];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) xop[rb][ks] = fld8(Xf + frag(rb, ks, KS, lane));
        // lane group g holds rows m0 + 16 g .. +15: their mask, max(mask, 0), 0 past M
        float mv[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int row = m0 + 16 * g + t;
            mv[t] = row < a.M ? fmaxf((float)a.mask[row], 0.f) : 0.f;
        }
        for (int cb = wave; cb < nb; cb += TW) {
            float4v ap[4], ag[4];
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                ap[rb] = float4v{0.f, 0.f, 0.f, 0.f};
                ag[rb] = float4v{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const half8 wp = fld8(Wp + frag(cb, ks, KS, lane));
                const half8 wg = fld8(Wg + frag(cb, ks, KS, lane));
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    ap[rb] = mfma16x16x32(xop[rb][ks], wp, ap[rb]);
                    ag[rb] = mfma16x16x32(xop[rb][ks], wg, ag[rb]);
                }
            }
            const int col = 16 * cb + r16;
            const float bpv = (float)a.bp[col], bgv = (float)a.bg[col];
            half_t* dst = (col < ci ? a.left + (int64_t)col * a.M : a.right + (int64_t)(col - ci) * a.M) +
                          m0 + 16 * g;
            half8 lo, hi;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 4 * rb + i;
                    const float v = mv[t] * (ap[rb][i] + bpv) * sigmoid_fast(ag[rb][i] + bgv);
                    if (t < 8) lo[t] = act_cvt<BF>(v); else hi[t - 8] = act_cvt<BF>(v);
                }
            const int rows_left = a.M - (m0 + 16 * g);
            if (vec && rows_left >= 16) {
                fst8_nt(dst, lo);
                fst8_nt(dst + 8, hi);
            } else {
#pragma unroll
                for (int t = 0; t < 16; ++t)
                    if (t < rows_left) dst[t] = t < 8 ? lo[t] : hi[t - 8];
            }
        }
    }
}

// The same op for M % 8 == 0 (16-byte channel-major stores), with a tile body that is straight-line
// code, so that no wait for a load also waits for the stores issued before it (vmcnt counts
// loads and stores in issue order, and the compiler's count is only as good as its weakest path):
// - the next tile's mask rows are fetched with its x rows, and the keep decision is taken from
//   them in registers (every wave's four lane groups hold all 64 rows, so a wave-wide any gives
//   the workgroup's decision without LDS or a barrier);
// - the loop is rotated so that the next tile's rows are fetched, the current tile's results
//   stored, and then the fetched rows waited for (keep decision, LayerNorm) in the same iteration;
// - every tile runs the LayerNorm and the GEMMs; a padding tile stores zeros, and the stores of a
//   skipped tile and of rows past M are buffer stores at an offset past the buffer's end, which
//   the hardware drops, so every tile issues the same stores and no branch skips them;
// - each wave owns CBW column blocks, fixed at compile time, with their biases in registers.
// Offsets are 32-bit: the launcher requires P/2 * M * 2 bytes < 2^31.
template <int K, int PH, int TH, bool BF>
__global__ __launch_bounds__(TH) void ln_gdp_fast_kernel(LnGdpArgs a) {
    constexpr int KS = K / 32, TW = TH / kWave, NB = PH / 8, CBW = NB / TW;
    static_assert(NB % TW == 0, "whole column blocks per wave");
    constexpr uint32_t kDrop = 0x80000000u;  // a store offset past every buffer's end
    using u32x4 = unsigned int __attribute__((ext_vector_type(4)));
    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    half_t* Wp = lds;
    half_t* Wg = Wp + 2 * PH * K;
    half_t* Xf = Wg + 2 * PH * K;
    float* sc = reinterpret_cast<float*>(Xf + kTileRows * K);
    float* of = sc + K;
    load_weight_frags<K, false>(Wp, a.wpT, 2 * PH, NB);
    load_weight_frags<K, false>(Wg, a.wgT, 2 * PH, NB);
    for (int i = threadIdx.x; i < K; i += TH) {
        sc[i] = a.scale[i];
        of[i] = a.offset[i];
    }
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform: scalar descriptors
    const int r16 = lane & 15, g = lane >> 4;
    const int tiles = (a.M + kTileRows - 1) / kTileRows;
    const int G = gridDim.x;
    const uint32_t out_bytes = (uint32_t)PH * (uint32_t)a.M * 2u;
    const auto rl = __builtin_amdgcn_make_buffer_rsrc(a.left, 0, out_bytes, 0x00020000);
    const auto rr = __builtin_amdgcn_make_buffer_rsrc(a.right, 0, out_bytes, 0x00020000);

    float bpv[CBW], bgv[CBW];
#pragma unroll
    for (int j = 0; j < CBW; ++j) {
        const int col = 16 * (wave + j * TW) + r16;
        bpv[j] = (float)a.bp[col];
        bgv[j] = (float)a.bg[col];
    }

    // rows of tile t (rows past M repeat row M - 1) and the mask of lane group g's 16 rows (the
    // 8-row chunks are all in or all out since M % 8 == 0; those past M are replaced at use)
    RowTile<K, kTileRows, TH> xt;
    half8 mlo, mhi;
    const auto fetch = [&](int t) {
        const int r0 = t * kTileRows + 16 * g;
        mlo = fld8(a.mask + min(r0, a.M - 8));
        mhi = fld8(a.mask + min(r0 + 8, a.M - 8));
        constexpr int TPR = RowTile<K, kTileRows, TH>::kTPR;
        const int row = threadIdx.x / TPR, part = threadIdx.x % TPR;
        const int m = min(t * kTileRows + row, a.M - 1);
#pragma unroll
        for (int j = 0; j < RowTile<K, kTileRows, TH>::kChunks; ++j)
            xt.v[j] = fld8(a.x + (int64_t)m * K + 8 * (part + TPR * j));
    };
    // the reference's keep rule for the tile (rows past M count as 0) and the rows' max(mask, 0)
    // (0 for NaN), on the fp16 pairs: an 8-row chunk is wholly inside M or past it; a row is live
    // if its max(mask, 0) is above 0, and the tile holds a zero if some mask has no magnitude bits
    typedef unsigned short ushort8 __attribute__((ext_vector_type(8)));
    half8 mvlo, mvhi;
    const auto decide = [&](int t) {
        const int r0 = t * kTileRows + 16 * g;
        const half8 klo = r0 < a.M ? mlo : fzero8(), khi = r0 + 8 < a.M ? mhi : fzero8();
        mvlo = __builtin_elementwise_max(klo, fzero8());
        mvhi = __builtin_elementwise_max(khi, fzero8());
        const bool live = __builtin_reduce_max(__builtin_elementwise_max(mvlo, mvhi)) > (half_t)0.f;
        const ushort8 mag = __builtin_elementwise_min(__builtin_bit_cast(ushort8, klo) & (unsigned short)0x7fff,
                                                      __builtin_bit_cast(ushort8, khi) & (unsigned short)0x7fff);
        const bool zero = __builtin_reduce_min(mag) == 0;
        const bool any_live = __any(live), any_zero = __any(zero);
        return any_live ? (int)kCompute : any_zero ? (int)kPadding : (int)kSkip;
    };
    const auto gemm_store = [&](int t, int work) {
        const int m0 = t * kTileRows;
        half8 xop[4][KS];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) xop[rb][ks] = fld8(Xf + frag(rb, ks, KS, lane));
        const bool zero_out = work == kPadding;
        const int rows_left = a.M - (m0 + 16 * g);  // <= 0, 8 or >= 16
        const bool st_lo = work != kSkip && rows_left >= 8, st_hi = work != kSkip && rows_left >= 16;
#pragma unroll
        for (int j = 0; j < CBW; ++j) {
            const int cb = wave + j * TW;
            // the products start from the biases
            float4v ap[4], ag[4];
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                ap[rb] = float4v{bpv[j], bpv[j], bpv[j], bpv[j]};
                ag[rb] = float4v{bgv[j], bgv[j], bgv[j], bgv[j]};
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const half8 wp = fld8(Wp + frag(cb, ks, KS, lane));
                const half8 wg = fld8(Wg + frag(cb, ks, KS, lane));
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    ap[rb] = mfma16x16x32(xop[rb][ks], wp, ap[rb]);
                    ag[rb] = mfma16x16x32(xop[rb][ks], wg, ag[rb]);
                }
            }
            half8 lo, hi;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int e = 4 * rb + i;
                    const float mv = (float)(e < 8 ? mvlo[e] : mvhi[e - 8]);
                    const float v = mv * ap[rb][i] * sigmoid_fast(ag[rb][i]);
                    if (e < 8) lo[e] = act_cvt<BF>(v); else hi[e - 8] = act_cvt<BF>(v);
                }
            if (zero_out) {
                lo = fzero8();
                hi = fzero8();
            }
            // column block cb lies wholly in left (columns < PH) or in right
            const int col = 16 * cb + r16;
            const bool is_left = 16 * cb < PH;
            const uint32_t off = ((uint32_t)(is_left ? col : col - PH) * (uint32_t)a.M + (uint32_t)(m0 + 16 * g)) * 2u;
            const auto rs = is_left ? rl : rr;
            // aux 2: nontemporal
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, lo), rs, st_lo ? off : kDrop, 0, 2);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, hi), rs, st_hi ? off + 16u : kDrop, 0, 2);
        }
    };

    int t = blockIdx.x;
    if (t >= tiles) return;
    fetch(t);
    int work = decide(t);
    __syncthreads();  // the weights and LayerNorm parameters are in LDS (decide has no barrier)
    ln_rows_to_frags<K, kTileRows, true, true, TH, BF>(Xf, xt, sc, of, a.eps);
    __syncthreads();
    for (;;) {
        const int nt = t + G;
        fetch(min(nt, tiles - 1));
        gemm_store(t, work);
        if (nt >= tiles) break;
        t = nt;
        work = decide(t);
        __syncthreads();  // every wave has read the previous tile's operands
        ln_rows_to_frags<K, kTileRows, true, true, TH, BF>(Xf, xt, sc, of, a.eps);
        __syncthreads();
    }
}

// ---- trimul_epilogue --------------------------------------------------------------------------

struct EpiArgs {
    const float* x_cm;  // [C][M]
    const half_t* x;    // [M][CA]
    const float *in_scale, *in_offset, *ln_scale, *ln_offset;
    const half_t *woT, *bo, *wgT, *bg;  // woT [O][C], wgT [O][CA]
    const half_t* keep;
    half_t* out;  // [M][O], may alias x with add_input
    int M, O;
    float eps;
};

// A wave's row tile, and the reference's keep unit for this op (cuda/volta_gdp.h:41), which two
// consecutive tiles share
constexpr int kEpiRows = 16;
constexpr int kEpiKeepRows = 32;

// LDS of the tri-mul epilogue: both weights, the LayerNorm parameters and the two bias vectors
constexpr size_t epi_lds_bytes(int C, int CA, int O) {
    return (size_t)(O * C + O * CA) * 2 + (size_t)(2 * C + 2 * CA + 2 * O) * 4;
}


// Each wave owns whole 16-row tiles and needs no other wave's data, so the tile loop has no
// barrier. Lane (r, g) holds row r of the tile, channels 32 ks + 8 g .. +7 of every contraction
// step ks: exactly the B operand of out^T = W Y^T, so both LayerNorms run in registers (a row's
// statistics summed over its four lanes by two xor shuffles) and write their fp16 output straight
// into the MFMA operands. The paired weight blocks in LDS give the lane 8 consecutive output
// columns of a column pair (a 16-byte store); the products start from the biases. Four waves per
// SIMD (at most 128 VGPRs): the weight reads of one column pair are in flight at a time.
// - The next tile's x_cm columns, x rows and keep values are fetched after this tile's
//   LayerNorms, so they are in flight during its products and stores; the loop waits for them
//   after the stores, so no fetched register crosses the back edge (vmcnt counts loads and stores
//   in issue order). With add_input the residual is this tile's x row, so the next one is fetched
//   after the stores.
// - Keep decisions come from a ballot of the 32 keep values of the tile's keep unit; padding
//   stores zeros, and the stores of skipped rows and rows past M go to an offset past the tile's
//   end, which the hardware drops, so no branch skips them.
template <int C, int CA, int O, bool ADD, bool BF>
__global__ __launch_bounds__(kEpiThreads, 4)
void epilogue_kernel(EpiArgs a) {
    constexpr int TW = kEpiThreads / kWave, KC = C / 32, KA = CA / 32, NP = O / 32;
    static_assert(!ADD || O == CA, "the residual is x itself");
    constexpr uint32_t kDrop = 0x80000000u;  // a store offset past every tile's end
    using u32x4 = unsigned int __attribute__((ext_vector_type(4)));
    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    half_t* Wo = lds;
    half_t* Wg = Wo + O * C;
    float* lsc = reinterpret_cast<float*>(Wg + O * CA);
    float* lof = lsc + C;
    float* isc = lof + C;
    float* iof = isc + CA;
    float* bov = iof + CA;
    float* bgv = bov + O;
    load_weight_frags<C, true>(Wo, a.woT, O, O / 16);
    load_weight_frags<CA, true>(Wg, a.wgT, O, O / 16);
    for (int i = threadIdx.x; i < C; i += kEpiThreads) {
        lsc[i] = a.ln_scale[i];
        lof[i] = a.ln_offset[i];
    }
    for (int i = threadIdx.x; i < CA; i += kEpiThreads) {
        isc[i] = a.in_scale[i];
        iof[i] = a.in_offset[i];
    }
    for (int i = threadIdx.x; i < O; i += kEpiThreads) {
        bov[i] = (float)a.bo[i];
        bgv[i] = (float)a.bg[i];
    }
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int r16 = lane & 15, g = lane >> 4;
    // the lane's LayerNorm parameters and biases, all at constant offsets from one address
    const float* prm = lsc + 8 * g;
    const int tiles = (a.M + kEpiRows - 1) / kEpiRows;
    const int stride = gridDim.x * TW;
    const bool has_keep = a.keep != nullptr;
    // without a keep the descriptor has no bytes, and its loads return zeros without touching memory
    const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.keep), 0,
                                                     has_keep ? (uint32_t)a.M * 2u : 0u, 0x00020000);

    // tile t's keep values (row m0k + lane % 32 of its keep unit), x_cm values and x row (rows
    // past M repeat row M - 1; their results are dropped)
    unsigned short kraw;
    float v[KC][8];
    half8 xr[KA];
    const auto fetch_cm = [&](int t) {
        const int m0 = t * kEpiRows, m0k = m0 & ~(kEpiKeepRows - 1);
        kraw = __builtin_amdgcn_raw_buffer_load_b16(rk, (uint32_t)min(m0k + (lane & 31), a.M - 1) * 2u, 0, 0);
        const float* pc = a.x_cm + (int64_t)(8 * g) * a.M + min(m0 + r16, a.M - 1);
#pragma unroll
        for (int ks = 0; ks < KC; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[ks][e] = pc[(int64_t)(32 * ks + e) * a.M];
    };
    const auto fetch_x = [&](int t) {
        const half_t* px = a.x + (int64_t)min(t * kEpiRows + r16, a.M - 1) * CA + 8 * g;
#pragma unroll
        for (int ks = 0; ks < KA; ++ks) xr[ks] = fld8(px + 32 * ks);
    };
    // the keep decision and both LayerNorms of tile t into the MFMA operands
    int work = kCompute;
    half8 yf[KC], af[KA];
    const auto prepare = [&](int t) {
        const int m0k = (t * kEpiRows) & ~(kEpiKeepRows - 1);
        const float k = m0k + (lane & 31) < a.M ? (has_keep ? (float)__builtin_bit_cast(half_t, kraw) : 1.f) : -1.f;
        const uint32_t live = (uint32_t)__ballot(k > 0.f), zero = (uint32_t)__ballot(k == 0.f);
        work = live ? (int)kCompute : zero ? (int)kPadding : (int)kSkip;
        {
            float s = 0.f;
#pragma unroll
            for (int ks = 0; ks < KC; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) s += v[ks][e];
            s += __shfl_xor(s, 16);
            s += __shfl_xor(s, 32);
            const float mean = s * (1.f / C);
            float q = 0.f;
#pragma unroll
            for (int ks = 0; ks < KC; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    v[ks][e] -= mean;
                    q += v[ks][e] * v[ks][e];
                }
            q += __shfl_xor(q, 16);
            q += __shfl_xor(q, 32);
            const float rstd = __builtin_amdgcn_rsqf(q * (1.f / C) + a.eps);
#pragma unroll
            for (int ks = 0; ks < KC; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    yf[ks][e] = (half_t)(v[ks][e] * rstd * prm[32 * ks + e] + prm[C + 32 * ks + e]);
        }
        __builtin_amdgcn_sched_barrier(0);
        {
            float s = 0.f;
#pragma unroll
            for (int ks = 0; ks < KA; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) s += act_get<BF>(xr[ks], e);
            s += __shfl_xor(s, 16);
            s += __shfl_xor(s, 32);
            const float mean = s * (1.f / CA);
            float q = 0.f;
#pragma unroll
            for (int ks = 0; ks < KA; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float d = act_get<BF>(xr[ks], e) - mean;
                    q += d * d;
                }
            q += __shfl_xor(q, 16);
            q += __shfl_xor(q, 32);
            const float rstd = __builtin_amdgcn_rsqf(q * (1.f / CA) + a.eps);
#pragma unroll
            for (int ks = 0; ks < KA; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    af[ks][e] = (half_t)((act_get<BF>(xr[ks], e) - mean) * rstd * prm[2 * C + 32 * ks + e] +
                                         prm[2 * C + CA + 32 * ks + e]);
        }
    };
    const auto gemm_store = [&](int t) {
        const int m0 = t * kEpiRows;
        // the tile's rows as one buffer: rows past M lie past its end
        const uint32_t rows = (uint32_t)min(kEpiRows, a.M - m0);
        const auto ro = __builtin_amdgcn_make_buffer_rsrc(a.out + (int64_t)m0 * O, 0, rows * O * 2u, 0x00020000);
        const bool store = work == kCompute || (!ADD && work == kPadding);
#pragma unroll
        for (int cp = 0; cp < NP; ++cp) {
            constexpr int kBo = 2 * C + 2 * CA, kBg = kBo + O;  // bov, bgv
            float4v ao[2], ag[2];
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                ao[hb] = *reinterpret_cast<const float4v*>(prm + kBo + 32 * cp + 4 * hb);
                ag[hb] = *reinterpret_cast<const float4v*>(prm + kBg + 32 * cp + 4 * hb);
            }
#pragma unroll
            for (int ks = 0; ks < KC; ++ks)
#pragma unroll
                for (int hb = 0; hb < 2; ++hb)
                    ao[hb] = mfma16x16x32(fld8(Wo + frag(2 * cp + hb, ks, KC, lane)), yf[ks], ao[hb]);
#pragma unroll
            for (int ks = 0; ks < KA; ++ks)
#pragma unroll
                for (int hb = 0; hb < 2; ++hb)
                    ag[hb] = mfma16x16x32(fld8(Wg + frag(2 * cp + hb, ks, KA, lane)), af[ks], ag[hb]);
            const int col = 32 * cp + 8 * g;
            half8 o;
            if (work == kPadding) {
                o = fzero8();
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float val = ao[j >> 2][j & 3] * sigmoid_fast(ag[j >> 2][j & 3]);
                    const float res = ADD ? pin_f32(act_get<BF>(xr[cp], j)) : 0.f;
                    o[j] = act_cvt<BF>(val + res);
                }
            }
            const uint32_t off = (uint32_t)(r16 * O + col) * 2u;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), ro, store ? off : kDrop, 0, 0);
            // one column pair's weight reads in flight at a time (hoisting them all costs registers)
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // With add_input the residual is this tile's x row, so the next tile's x row is fetched only
    // after this tile's stores (the output aliases x, but the next tile's rows are not this one's).
    int t = blockIdx.x * TW + wave;
    fetch_cm(min(t, tiles - 1));
    fetch_x(min(t, tiles - 1));
    __syncthreads();  // the weights, LayerNorm parameters and biases are in LDS
    if (t >= tiles) return;
    prepare(t);
    for (;;) {
        const int nt = t + stride;
        fetch_cm(min(nt, tiles - 1));
        if constexpr (!ADD) fetch_x(min(nt, tiles - 1));
        gemm_store(t);
        if (nt >= tiles) break;
        if constexpr (ADD) fetch_x(nt);
        t = nt;
        prepare(t);
    }
}

// ---- transition -------------------------------------------------------------------------------
//
// out^T = W2^T relu(W1 X^T + b1) + b2 over hidden chunks of 64: the first product's accumulator
// (rows = hidden units in pair order) is exactly the B operand of the second, so the hidden
// activation never leaves registers. At C = 128 and 256 the weights do not fit in LDS whole, so
// 64-unit chunks stream through it (each through registers into one buffer between two barriers)
// and every weight fragment a wave reads feeds one MFMA per 16-row block of its rows: at C = 128 a
// 256-row tile (two blocks a wave, which halves the LDS weight reads per MFMA: the kernel is bound
// by them), at C = 256 128 rows. The biases live in LDS, so no global load is waited for between a
// chunk's prefetch and its use; the last chunk prefetches the first for the next tile. At C = 64
// both weights fit in LDS, and transition_rows_kernel below serves that width.
constexpr int kHid = 64;
template <int C>
constexpr int trans_rows() { return C == 128 ? 256 : 128; }

struct TransArgs {
    const half_t* x;
    const float *scale, *offset;
    const half_t *w1T, *b1, *w2T, *b2;  // w1T [H][C], w2T [H/64][C][64]
    const half_t* keep;
    half_t* out;
    int M, H;
    float eps;
};

template <int C>
struct TransTile {
    static constexpr int KS = C / 32;
    static constexpr int kW1 = 4 * KS * kWave * 8;        // halfs: 4 hidden blocks
    static constexpr int kW2 = (C / 16) * 2 * kWave * 8;  // halfs: C/16 blocks x 2 steps
    static constexpr int kChunks = (kW1 + kW2) / 8;
    static constexpr int kCPT = kChunks / kFThreads;
    static constexpr int kSub = C > 128 ? 32 : 64;        // keep granularity (volta_ops.cu:551-553)
};

// Threads per workgroup (one workgroup per CU): at C = 128 eight waves of two 16-row blocks, at
// C = 256 four waves of two row blocks.
constexpr int trans_threads(int C) { return C <= 128 ? 512 : 256; }

template <int C, bool ADD, int TH, bool BF>
__global__ __launch_bounds__(TH, TH / 256) void transition_kernel(TransArgs a) {
    using T = TransTile<C>;
    constexpr int kTR = trans_rows<C>();
    constexpr int TW = TH / kWave, RB = kTR / 16 / TW, kCPT = T::kChunks / TH;
    static_assert(RB * TW * 16 == kTR && kCPT * TH == T::kChunks, "whole row blocks and chunks");
    constexpr int KS = T::KS, NCB = C / 16, NSUB = kTR / T::kSub;
    static_assert(C != 64, "C = 64 is transition_rows_kernel's");
    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    half_t* Xf = lds;                   // the row tile's LayerNorm output, fragment-major
    half_t* W1 = Xf + kTR * C;          // (C = 256) hidden chunk of w1, then of w2
    half_t* W2 = W1 + T::kW1;
    float* sc = reinterpret_cast<float*>(W2 + T::kW2);
    float* of = sc + C;
    float* b2s = of + C;
    float* b1s = b2s + C;  // [H]
    for (int i = threadIdx.x; i < C; i += TH) {
        sc[i] = a.scale[i];
        of[i] = a.offset[i];
        b2s[i] = a.b2[i];
    }
    for (int i = threadIdx.x; i < a.H; i += TH) b1s[i] = a.b1[i];
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int r16 = lane & 15, g = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int tiles = (a.M + kTR - 1) / kTR;
    const int chunks = a.H / kHid;

    // weight chunk j: W1 fragments of hidden rows 64 j + pair_row(hb, r), W2 fragments of output
    // channels pair_row(cb, r) over hidden 64 j + 32 kt + 8 g ..; fragment t (of 64 lanes' 16-byte
    // operands) is 16-byte chunks 64 t .. + 63 of the chunk, and thread i stages chunk i
    half8 wreg[kCPT];
    const auto fetch_w = [&](int j) {
#pragma unroll
        for (int u = 0; u < kCPT; ++u) {
            const int i = threadIdx.x + u * TH;
            const int l = i % kWave, t = i / kWave;
            if (i < T::kW1 / 8) {
                const int ks = t % KS, hb = t / KS;
                const int hid = kHid * j + pair_row(hb, l & 15);
                wreg[u] = fld8(a.w1T + (int64_t)hid * C + 32 * ks + 8 * (l >> 4));
            } else {
                const int t2 = t - T::kW1 / (8 * kWave);
                const int kt = t2 & 1, cb = t2 >> 1;
                const int c = pair_row(cb, l & 15);
                wreg[u] = fld8(a.w2T + ((int64_t)j * C + c) * kHid + 32 * kt + 8 * (l >> 4));
            }
        }
    };
    const auto store_w = [&]() {
#pragma unroll
        for (int u = 0; u < kCPT; ++u) fst8(W1 + (threadIdx.x + u * TH) * 8, wreg[u]);
    };

    RowTile<C, kTR, TH> xt;
    fetch_w(0);
    for (int tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
        const int m0 = tile * kTR;
        int work[NSUB];
        bool any = false;
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            work[s] = tile_work(a.keep, a.M, m0 + s * T::kSub, T::kSub, -1.f);
            any |= work[s] == kCompute;
        }
        if (!any) {
            if (!ADD) {
                for (int i = threadIdx.x; i < kTR * C / 8; i += TH) {
                    const int r = i / (C / 8), c = (i % (C / 8)) * 8;
                    if (work[r / T::kSub] == kPadding && m0 + r < a.M)
                        fst8(a.out + (int64_t)(m0 + r) * C + c, fzero8());
                }
            }
            continue;
        }
        fetch_rows<C, kTR>(xt, a.x, a.M, m0);
        __syncthreads();
        ln_rows_to_frags<C, kTR, false, true, TH, BF>(Xf, xt, sc, of, a.eps);

        float4v acc[NCB][RB];
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) acc[cb][rb] = float4v{0.f, 0.f, 0.f, 0.f};
        half8 xop[RB][KS];
        for (int j = 0; j < chunks; ++j) {
            __syncthreads();  // the previous chunk's weight reads are done
            store_w();
            __syncthreads();
            if (j == 0) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) xop[rb][ks] = fld8(Xf + frag(RB * wave + rb, ks, KS, lane));
            }
            fetch_w(j + 1 < chunks ? j + 1 : 0);  // the first chunk again for the next tile

            // hidden^T for 64 units x this wave's 16 RB rows
            float4v hacc[4][RB];
#pragma unroll
            for (int hb = 0; hb < 4; ++hb)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) hacc[hb][rb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int hb = 0; hb < 4; ++hb) {
                    const half8 w = fld8(W1 + frag(hb, ks, KS, lane));
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) hacc[hb][rb] = mfma16x16x32(w, xop[rb][ks], hacc[hb][rb]);
                }
            }
            half8 hop[2][RB];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                float b1v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) b1v[e] = b1s[kHid * j + 32 * kt + 8 * g + e];
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        hop[kt][rb][e] = (half_t)fmaxf(hacc[2 * kt + (e >> 2)][rb][e & 3] + b1v[e], 0.f);
            }
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) {
                    const half8 w = fld8(W2 + frag(cb, kt, 2, lane));
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) acc[cb][rb] = mfma16x16x32(w, hop[kt][rb], acc[cb][rb]);
                }
            }
        }

        // lane: channels 32 (cb/2) + 8 g .. +7 of rows m0 + 16 (RB wave + rb) + r16
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int lr = 16 * (RB * wave + rb) + r16, row = m0 + lr;
            const int w = work[lr / T::kSub];
            if (row >= a.M || w == kSkip || (ADD && w == kPadding)) continue;
#pragma unroll
            for (int cp = 0; cp < NCB / 2; ++cp) {
                const int col = 32 * cp + 8 * g;
                half_t* dst = a.out + (int64_t)row * C + col;
                if (w == kPadding) {
                    fst8(dst, fzero8());
                    continue;
                }
                const half8 xa = ADD ? fld8(a.x + (int64_t)row * C + col) : fzero8();
                half8 o;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    o[e] = act_cvt<BF>(acc[2 * cp + (e >> 2)][rb][e & 3] + b2s[col + e] + act_get<BF>(xa, e));
                fst8(dst, o);
            }
        }
    }
}

// The transition at C = 64, where both weights fit in LDS at once (W1 [H][64] and W2 [64][H], at
// most 64 KB): one workgroup of 16 waves per CU holds them for the whole call, and each wave owns
// whole 32-row tiles (two 16-row blocks), so the tile loop has no barrier. As in the tri-mul
// epilogue, lane (r, g) loads exactly its B-operand slots of x (row r of each block, channels
// 32 ks + 8 g .. +7), runs the LayerNorm in registers (a row's statistics over its four lanes by two
// xor shuffles) and keeps the fp16 result as the first product's operand. The hidden units go 32
// at a time: two paired W1 blocks give the lane hidden units 32 p + 8 g .. +7 of its rows, which
// after bias, relu and rounding to fp16 are exactly its B operand of the second product's step p,
// so the hidden activation never leaves registers. Every weight fragment read feeds both blocks.
// - The next tile's x rows and keep values are fetched after this tile's LayerNorm (with
//   add_input, whose residual is this tile's x, after its stores), so no fetched register crosses
//   the back edge (vmcnt counts loads and stores in issue order).
// - Keep decisions come from a ballot of the 64 keep values of the tile's keep unit (64 rows at
//   C = 64, cuda/volta_ops.cu:551-553); padding stores zeros, and the stores of skipped rows and
//   rows past M go to an offset past the tile's end, which the hardware drops.
constexpr int kTransRowsThreads = 1024;
constexpr int kTransRowsTile = 32;
constexpr size_t trans_rows_lds_bytes(int C, int H) { return (size_t)2 * H * C * 2 + (size_t)(3 * C + H) * 4; }

template <bool ADD, bool BF>
__global__ __launch_bounds__(kTransRowsThreads, 4) void transition_rows_kernel(TransArgs a) {
    constexpr int C = 64, KS = C / 32, NCB = C / 16, RB = kTransRowsTile / 16, TW = kTransRowsThreads / kWave;
    constexpr int kKeep = TransTile<C>::kSub;
    constexpr uint32_t kDrop = 0x80000000u;  // a store offset past every tile's end
    using u32x4 = unsigned int __attribute__((ext_vector_type(4)));
    extern __shared__ __attribute__((aligned(16))) half_t lds[];
    const int H = a.H, KH = H / 32;
    half_t* W1 = lds;          // [H/16 paired blocks][KS][64 lanes][8]
    half_t* W2 = W1 + H * C;   // [C/16 paired blocks][KH][64 lanes][8]
    float* sc = reinterpret_cast<float*>(W2 + H * C);
    float* of = sc + C;
    float* b2s = of + C;
    float* b1s = b2s + C;  // [H]
    load_weight_frags<C, true>(W1, a.w1T, H, H / 16);
    // W2 operand block cb, step p: output channels pair_row(cb, r), hidden 32 p + 8 g .. +7, from
    // the blocked w2T [H/64][C][64]
    for (int i = threadIdx.x; i < NCB * KH * kWave; i += kTransRowsThreads) {
        const int l = i % kWave, t = i / kWave, p = t % KH, cb = t / KH;
        const int c = pair_row(cb, l & 15);
        fst8(W2 + i * 8, fld8(a.w2T + ((int64_t)(p >> 1) * C + c) * kHid + 32 * (p & 1) + 8 * (l >> 4)));
    }
    for (int i = threadIdx.x; i < C; i += kTransRowsThreads) {
        sc[i] = a.scale[i];
        of[i] = a.offset[i];
        b2s[i] = a.b2[i];
    }
    for (int i = threadIdx.x; i < H; i += kTransRowsThreads) b1s[i] = a.b1[i];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int r16 = lane & 15, g = lane >> 4;
    const int tiles = (a.M + kTransRowsTile - 1) / kTransRowsTile;
    const int stride = gridDim.x * TW;
    const bool has_keep = a.keep != nullptr;
    // without a keep the descriptor has no bytes, and its loads return zeros without touching memory
    const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.keep), 0,
                                                     has_keep ? (uint32_t)a.M * 2u : 0u, 0x00020000);

    // tile t's keep values (row m0k + lane of its keep unit) and x rows (rows past M repeat row
    // M - 1; their results are dropped)
    unsigned short kraw;
    half8 xr[RB][KS];
    const auto fetch = [&](int t) {
        const int m0 = t * kTransRowsTile, m0k = m0 & ~(kKeep - 1);
        kraw = __builtin_amdgcn_raw_buffer_load_b16(rk, (uint32_t)min(m0k + lane, a.M - 1) * 2u, 0, 0);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const half_t* px = a.x + (int64_t)min(m0 + 16 * rb + r16, a.M - 1) * C + 8 * g;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) xr[rb][ks] = fld8(px + 32 * ks);
        }
    };
    int work = kCompute;
    half8 yf[RB][KS];
    const auto prepare = [&](int t) {
        const int m0k = (t * kTransRowsTile) & ~(kKeep - 1);
        const float k = m0k + lane < a.M ? (has_keep ? (float)__builtin_bit_cast(half_t, kraw) : 1.f) : -1.f;
        const uint64_t live = __ballot(k > 0.f), zero = __ballot(k == 0.f);
        work = live ? (int)kCompute : zero ? (int)kPadding : (int)kSkip;
        const float* prm = sc + 8 * g;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            float s = 0.f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) s += act_get<BF>(xr[rb][ks], e);
            s += __shfl_xor(s, 16);
            s += __shfl_xor(s, 32);
            const float mean = s * (1.f / C);
            float q = 0.f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float d = act_get<BF>(xr[rb][ks], e) - mean;
                    q += d * d;
                }
            q += __shfl_xor(q, 16);
            q += __shfl_xor(q, 32);
            const float rstd = __builtin_amdgcn_rsqf(q * (1.f / C) + a.eps);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    yf[rb][ks][e] = (half_t)((act_get<BF>(xr[rb][ks], e) - mean) * rstd * prm[32 * ks + e] +
                                             prm[C + 32 * ks + e]);
        }
    };
    const auto gemm_store = [&](int t) {
        // both products start from their biases: paired block b gives lane group g the rows
        // 32 (b / 2) + 8 g + 4 (b % 2) .. +3 (output channels of W2's blocks, hidden units of W1's)
        float4v acc[NCB][RB];
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
            const float4v b2q = *reinterpret_cast<const float4v*>(b2s + 32 * (cb >> 1) + 8 * g + 4 * (cb & 1));
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) acc[cb][rb] = b2q;
        }
        const float* b1l = b1s + 8 * g;
        for (int p = 0; p < KH; ++p) {
            float4v hacc[2][RB];
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const float4v b1q = *reinterpret_cast<const float4v*>(b1l + 32 * p + 4 * h2);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) hacc[h2][rb] = b1q;
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    const half8 w = fld8(W1 + frag(2 * p + h2, ks, KS, lane));
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) hacc[h2][rb] = mfma16x16x32(w, yf[rb][ks], hacc[h2][rb]);
                }
            // (one product's fragment reads in flight at a time: hoisting more costs registers)
            __builtin_amdgcn_sched_barrier(0);
            // relu, fp16: slot 8 g + e of step p is hidden unit 32 p + 8 g + e
            half8 hop[RB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                for (int e = 0; e < 8; ++e) hop[rb][e] = (half_t)fmaxf(hacc[e >> 2][rb][e & 3], 0.f);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                const half8 w = fld8(W2 + frag(cb, p, KH, lane));
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) acc[cb][rb] = mfma16x16x32(w, hop[rb], acc[cb][rb]);
            }
        }
        // lane: channels 32 cp + 8 g .. +7 of rows m0 + 16 rb + r16
        const int m0 = t * kTransRowsTile;
        const uint32_t rows = (uint32_t)min(kTransRowsTile, a.M - m0);
        const auto ro = __builtin_amdgcn_make_buffer_rsrc(a.out + (int64_t)m0 * C, 0, rows * C * 2u, 0x00020000);
        const bool store = work == kCompute || (!ADD && work == kPadding);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int cp = 0; cp < NCB / 2; ++cp) {
                const int col = 32 * cp + 8 * g;
                half8 o;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float res = ADD ? act_get<BF>(xr[rb][cp], e) : 0.f;
                    o[e] = act_cvt<BF>(acc[2 * cp + (e >> 2)][rb][e & 3] + res);
                }
                // a padding tile stores zeros (with add_input it stores nothing)
                const u32x4 ov = !ADD && work == kPadding ? u32x4{0u, 0u, 0u, 0u} : __builtin_bit_cast(u32x4, o);
                const uint32_t off = (uint32_t)((16 * rb + r16) * C + col) * 2u;
                __builtin_amdgcn_raw_buffer_store_b128(ov, ro, store ? off : kDrop, 0, 0);
            }
    };

    int t = blockIdx.x * TW + wave;
    fetch(min(t, tiles - 1));
    __syncthreads();  // the weights, LayerNorm parameters and biases are in LDS
    if (t >= tiles) return;
    prepare(t);
    for (;;) {
        const int nt = t + stride;
        if constexpr (!ADD) fetch(min(nt, tiles - 1));
        gemm_store(t);
        if (nt >= tiles) break;
        if constexpr (ADD) fetch(nt);
        t = nt;
        prepare(t);
    }
}

// ---- host side --------------------------------------------------------------------------------

static int fused_cu_count() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) {
            cus = v;
        } else {
            cus = 256;
        }
    }
    return cus;
}

static int fused_lds_limit() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    return shared_limit(dev);
}

template <typename F>
static int launch_fused(const char* what, F kernel, dim3 grid, size_t lds, hipStream_t s,
                        const void* args_ptr, size_t) {
    (void)args_ptr;
    const int limit = fused_lds_limit();
    if (limit > 0 && lds > (size_t)limit) {
        return invalid(std::string(what) + ": needs " + std::to_string(lds / 1024) +
                       " KB shared, device allows " + std::to_string(limit / 1024) + " KB");
    }
    if (lds > 64 * 1024) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    }
    (void)grid;
    (void)s;
    return CLK_OK;
}

static bool fused_width(int64_t c) { return c == 64 || c == 128; }
static bool msa_width(int64_t c) { return fused_width(c) || c == 256; }

static unsigned persistent_grid(int64_t tiles, size_t lds, int max_per_cu = 4) {
    const int limit = fused_lds_limit();
    int per_cu = std::min(2, max_per_cu);
    if (limit > 0 && lds > 0) per_cu = std::max(1, std::min(max_per_cu, (int)(limit / lds)));
    const int64_t g = std::min<int64_t>(tiles, (int64_t)fused_cu_count() * per_cu);
    return (unsigned)std::max<int64_t>(g, 1);
}

}  // namespace clk

using namespace clk;

static const half_t* f16p(const clk_buffer* b) { return static_cast<const half_t*>(b->data); }
static const float* f32p(const clk_buffer* b) { return static_cast<const float*>(b->data); }

template <bool BF>
static int ln_gdp_launch(const LnGdpArgs& a, int64_t M, int64_t K, int64_t P, hipStream_t s) {
    const size_t lds = (size_t)(2 * P * K + kTileRows * K) * 2 + 2 * K * 4;
    const int64_t tiles = (M + kTileRows - 1) / kTileRows;
    const dim3 grid(persistent_grid(tiles, lds));
    if (M % 8 == 0 && P / 2 * M * 2 < (int64_t{1} << 31)) {  // 16-byte channel-major stores, 32-bit offsets
#define CLK_GDP_FAST(K_, PH_)                                                                          \
    if (K == K_ && P / 2 == PH_) {                                                                     \
        const auto kern = ln_gdp_fast_kernel<K_, PH_, gdp_threads<K_>(), BF>;                          \
        if (int st = launch_fused("ln_gdp", kern, grid, lds, s, &a, 0)) return st;                     \
        stage_mark(s, 0);                                                                              \
        hipLaunchKernelGGL(kern, grid, dim3(gdp_threads<K_>()), lds, s, a);                            \
        stage_mark(s, 1);                                                                              \
        return launch_status("ln_gdp");                                                                \
    }
        CLK_GDP_FAST(64, 64) CLK_GDP_FAST(64, 128) CLK_GDP_FAST(128, 64) CLK_GDP_FAST(128, 128)
#undef CLK_GDP_FAST
    }
    if (K == 64) {
        if (int st = launch_fused("ln_gdp", ln_gdp_kernel<64, gdp_threads<64>(), BF>, grid, lds, s, &a, 0)) return st;
        stage_mark(s, 0);
        hipLaunchKernelGGL((ln_gdp_kernel<64, gdp_threads<64>(), BF>), grid, dim3(gdp_threads<64>()), lds, s, a);
        stage_mark(s, 1);
    } else {
        if (int st = launch_fused("ln_gdp", ln_gdp_kernel<128, gdp_threads<128>(), BF>, grid, lds, s, &a, 0)) return st;
        stage_mark(s, 0);
        hipLaunchKernelGGL((ln_gdp_kernel<128, gdp_threads<128>(), BF>), grid, dim3(gdp_threads<128>()), lds, s, a);
        stage_mark(s, 1);
    }
    return launch_status("ln_gdp");
}

// The activation type of a fused call: fp16 (the reference's contract) or bf16, one for all of
// the call's activation buffers (`acts`); CLK_F16 if the first is neither, so the type check
// reports it.
static int act_type(const clk_buffer* first) {
    return first != nullptr && first->dtype == CLK_BF16 ? CLK_BF16 : CLK_F16;
}

// The type an optional activation buffer must have: the call's activation type when it is used;
// an unused one-element stand-in may be F16 or BF16.
static int opt_act_type(const clk_buffer* b, bool used, int at) {
    if (used || b == nullptr) return at;
    return b->dtype == CLK_F16 || b->dtype == CLK_BF16 ? b->dtype : at;
}

extern "C" int clk_ln_gdp(clk_stream stream, const clk_buffer* x, const clk_buffer* scale,
                          const clk_buffer* offset, const clk_buffer* wpT, const clk_buffer* bp,
                          const clk_buffer* wgT, const clk_buffer* bg, const clk_buffer* mask,
                          const clk_buffer* left, const clk_buffer* right, float eps) {
    const clk_buffer* bufs[] = {x, scale, offset, wpT, bp, wgT, bg, mask, left, right};
    const int at = act_type(x);
    const int types[] = {at, CLK_F32, CLK_F32, CLK_F16, CLK_F16, CLK_F16, CLK_F16, CLK_F16, at, at};
    if (int st = check_types("ln_gdp", bufs, types, 10)) return st;
    if (x->rank != 2 || wpT->rank != 2 || wpT->dims[1] != x->dims[1]) {
        return invalid("ln_gdp: x must be [M,K] and wpT [P,K]");
    }
    const int64_t M = x->dims[0], K = x->dims[1], P = wpT->dims[0];
    if (!fused_width(K) || P % 2 || !fused_width(P / 2)) return invalid("ln_gdp: K and P/2 must be 64 or 128");
    if (elements(wgT) != P * K || elements(bp) != P || elements(bg) != P || elements(mask) != M ||
        elements(left) != P / 2 * M || elements(right) != P / 2 * M || elements(scale) != K ||
        elements(offset) != K) {
        return invalid("ln_gdp: shapes do not match x [M,K], wpT [P,K]");
    }
    if (M == 0) return ok();
    if (!aligned16(x->data) || !aligned16(wpT->data) || !aligned16(wgT->data) || !aligned16(left->data) ||
        !aligned16(right->data) || !aligned16(mask->data)) {
        return invalid("ln_gdp: x, weights, mask and results must be 16-byte aligned");
    }
    LnGdpArgs a{f16p(x), f32p(scale), f32p(offset), f16p(wpT), f16p(bp), f16p(wgT), f16p(bg), f16p(mask),
                static_cast<half_t*>(left->data), static_cast<half_t*>(right->data), (int)M, (int)P, eps};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    return at == CLK_BF16 ? ln_gdp_launch<true>(a, M, K, P, s) : ln_gdp_launch<false>(a, M, K, P, s);
}

template <int C, int CA, int O, bool ADD, bool BF>
static int run_epilogue(const EpiArgs& a, hipStream_t s) {
    constexpr int TH = kEpiThreads;
    constexpr size_t lds = epi_lds_bytes(C, CA, O);
    // one 16-row tile per wave at a time; one workgroup of 16 waves per CU (four per SIMD, the
    // kernel's launch bounds), measured 1-3% faster than two of eight, which each load the weights
    const int64_t groups = ((a.M + kEpiRows - 1) / kEpiRows + TH / kWave - 1) / (TH / kWave);
    const dim3 grid(persistent_grid(groups, lds, 4 * 4 / (TH / kWave)));
    if (int st = launch_fused("trimul_epilogue", epilogue_kernel<C, CA, O, ADD, BF>, grid, lds, s, &a, 0)) return st;
    stage_mark(s, 0);
    hipLaunchKernelGGL((epilogue_kernel<C, CA, O, ADD, BF>), grid, dim3(TH), lds, s, a);
    stage_mark(s, 1);
    return launch_status("trimul_epilogue");
}

template <int C, int CA, bool BF>
static int epilogue_dispatch_o(const EpiArgs& a, bool add, hipStream_t s) {
    if (add) return run_epilogue<C, CA, CA, true, BF>(a, s);  // add_input implies O == CA (checked above)
    return a.O == 64 ? run_epilogue<C, CA, 64, false, BF>(a, s) : run_epilogue<C, CA, 128, false, BF>(a, s);
}

template <int C, bool BF>
static int epilogue_dispatch(const EpiArgs& a, int64_t CA, bool add, hipStream_t s) {
    return CA == 64 ? epilogue_dispatch_o<C, 64, BF>(a, add, s) : epilogue_dispatch_o<C, 128, BF>(a, add, s);
}

extern "C" int clk_trimul_epilogue(clk_stream stream, const clk_buffer* x_cm, const clk_buffer* x,
                                   const clk_buffer* in_scale, const clk_buffer* in_offset,
                                   const clk_buffer* ln_scale, const clk_buffer* ln_offset,
                                   const clk_buffer* woT, const clk_buffer* bo, const clk_buffer* wgT,
                                   const clk_buffer* bg, const clk_buffer* keep, const clk_buffer* out,
                                   float eps, int32_t add_input, int32_t has_keep) {
    const clk_buffer* bufs[] = {x_cm, x, in_scale, in_offset, ln_scale, ln_offset, woT, bo, wgT, bg, keep, out};
    const int at = act_type(x);
    const int types[] = {CLK_F32, at, CLK_F32, CLK_F32, CLK_F32, CLK_F32,
                         CLK_F16, CLK_F16, CLK_F16, CLK_F16, CLK_F16, at};
    if (int st = check_types("trimul_epilogue", bufs, types, 12)) return st;
    if (x_cm->rank != 2 || x->rank != 2 || woT->rank != 2 || x->dims[0] != x_cm->dims[1] ||
        woT->dims[1] != x_cm->dims[0]) {
        return invalid("trimul_epilogue: x_cm [C,M], x [M,CA], woT [O,C]");
    }
    const int64_t C = x_cm->dims[0], M = x_cm->dims[1], CA = x->dims[1], O = woT->dims[0];
    if (!fused_width(C) || !fused_width(CA) || !fused_width(O) || (add_input && O != CA)) {
        return invalid("trimul_epilogue: C, CA and O must be 64 or 128, O == CA with add_input");
    }
    if (elements(wgT) != O * CA || elements(bo) != O || elements(bg) != O || elements(in_scale) != CA ||
        elements(in_offset) != CA || elements(ln_scale) != C || elements(ln_offset) != C ||
        elements(out) != M * O || (has_keep && elements(keep) != M)) {
        return invalid("trimul_epilogue: shapes do not match");
    }
    if (M == 0) return ok();
    if (!aligned16(x->data) || !aligned16(woT->data) || !aligned16(wgT->data) || !aligned16(out->data)) {
        return invalid("trimul_epilogue: x, weights and out must be 16-byte aligned");
    }
    EpiArgs a{f32p(x_cm), f16p(x), f32p(in_scale), f32p(in_offset), f32p(ln_scale), f32p(ln_offset),
              f16p(woT), f16p(bo), f16p(wgT), f16p(bg), has_keep ? f16p(keep) : nullptr,
              static_cast<half_t*>(out->data), (int)M, (int)O, eps};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (at == CLK_BF16) {
        return C == 64 ? epilogue_dispatch<64, true>(a, CA, add_input, s)
                       : epilogue_dispatch<128, true>(a, CA, add_input, s);
    }
    return C == 64 ? epilogue_dispatch<64, false>(a, CA, add_input, s)
                   : epilogue_dispatch<128, false>(a, CA, add_input, s);
}

template <int K, bool LN, bool BF>
static int run_proj(const ProjArgs& a0, hipStream_t s, const char* what) {
    ProjArgs a = a0;
    // columns per workgroup: all of them while the weights fit beside the tile in LDS
    const int limit = fused_lds_limit();
    const size_t fixed = (size_t)(16 * K + kTileRows * K) * 2 + 2 * K * 4;
    int cols = a.n;
    if (limit > 0) {
        while (cols > 32 && fixed + (size_t)cols * K * 2 > (size_t)limit) cols = (cols / 2 + 31) / 32 * 32;
    }
    a.cols = std::max(cols, 32);
    const int chunks = a.n > 0 ? (a.n + a.cols - 1) / a.cols : 1;
    const size_t lds = (size_t)(std::min(a.cols, std::max(a.n, 0)) * K) * 2 + fixed;
    const int64_t tiles = (a.M + kTileRows - 1) / kTileRows;
    const dim3 grid(persistent_grid(tiles, lds), chunks);
    constexpr int TH = kProjThreads, TW = TH / kWave;
    // the fixed-shape kernel: no keep mask, and every column chunk a whole number (1 or 2) of
    // column pairs per wave
    if constexpr (LN) {
        // whole-row stores: the weights in registers, the output tile staged in LDS
        if (a.keep == nullptr && (a.n == 256 || a.n == 512) && a.heads <= 16) {
            const size_t rlds = (size_t)(kTileRows * a.n + kTileRows * K + 16 * K) * 2 + 2 * K * 4;
            const dim3 rgrid(persistent_grid(tiles, rlds, K == 64 ? 2 : 1));
#define CLK_PROJ_ROWS(N_)                                                                              \
            if (a.n == N_) {                                                                           \
                if (int st = launch_fused(what, proj_rows_kernel<K, N_, BF>, rgrid, rlds, s, &a, 0)) return st; \
                stage_mark(s, 0);                                                                      \
                hipLaunchKernelGGL((proj_rows_kernel<K, N_, BF>), rgrid, dim3(kProjThreads), rlds, s, a); \
                stage_mark(s, 1);                                                                      \
                return launch_status(what);                                                            \
            }
            CLK_PROJ_ROWS(256) CLK_PROJ_ROWS(512)
#undef CLK_PROJ_ROWS
        }
    }
    const int pairs = a.cols / 32;
    const bool fast = a.keep == nullptr && a.n % a.cols == 0 && pairs % TW == 0 &&
                      (pairs / TW == 1 || pairs / TW == 2);
    if (fast && pairs / TW == 1) {
        if (int st = launch_fused(what, proj_fast_kernel<K, LN, TH, 1, BF>, grid, lds, s, &a, 0)) return st;
    } else if (fast) {
        if (int st = launch_fused(what, proj_fast_kernel<K, LN, TH, 2, BF>, grid, lds, s, &a, 0)) return st;
    } else {
        if (int st = launch_fused(what, proj_kernel<K, LN, TH, BF>, grid, lds, s, &a, 0)) return st;
    }
    stage_mark(s, 0);
    if (fast && pairs / TW == 1) {
        hipLaunchKernelGGL((proj_fast_kernel<K, LN, TH, 1, BF>), grid, dim3(TH), lds, s, a);
    } else if (fast) {
        hipLaunchKernelGGL((proj_fast_kernel<K, LN, TH, 2, BF>), grid, dim3(TH), lds, s, a);
    } else {
        hipLaunchKernelGGL((proj_kernel<K, LN, TH, BF>), grid, dim3(TH), lds, s, a);
    }
    stage_mark(s, 1);
    return launch_status(what);
}

template <int K, int N, bool RES, bool BF>
static int run_outproj(const ProjArgs& a, hipStream_t s) {
    constexpr size_t lds = (size_t)(N * K + kTileRows * K) * 2;
    const int64_t tiles = (a.M + kTileRows - 1) / kTileRows;
    // two workgroups per CU: the registers the kernel is compiled for allow no more
    const dim3 grid(persistent_grid(tiles, lds, 2));
    if (int st = launch_fused("output_projection", outproj_kernel<K, N, RES, BF>, grid, lds, s, &a, 0)) return st;
    stage_mark(s, 0);
    hipLaunchKernelGGL((outproj_kernel<K, N, RES, BF>), grid, dim3(kProjThreads), lds, s, a);
    stage_mark(s, 1);
    return launch_status("output_projection");
}

extern "C" int clk_ln_projection(clk_stream stream, const clk_buffer* x, const clk_buffer* scale,
                                 const clk_buffer* offset, const clk_buffer* wT, const clk_buffer* wbT,
                                 const clk_buffer* keep, const clk_buffer* p, const clk_buffer* bias,
                                 float eps, int64_t n, int64_t heads, int32_t has_keep) {
    const clk_buffer* bufs[] = {x, scale, offset, wT, wbT, keep, p, bias};
    const int at = act_type(x);
    const int types[] = {at, CLK_F32, CLK_F32, CLK_F16, CLK_F16, CLK_F16, opt_act_type(p, n > 0, at),
                         opt_act_type(bias, heads > 0, at)};
    if (int st = check_types("ln_projection", bufs, types, 8)) return st;
    if (x->rank != 2) return invalid("ln_projection: x must be [M,K]");
    const int64_t M = x->dims[0], K = x->dims[1];
    if (!fused_width(K) || n < 0 || n % 64 || heads < 0 || heads > 8) {
        return invalid("ln_projection: K must be 64 or 128, n a multiple of 64, at most 8 heads");
    }
    if (elements(scale) != K || elements(offset) != K ||
        (n && (elements(wT) != n * K || elements(p) != M * n)) ||
        (heads && (elements(wbT) != heads * K || elements(bias) != heads * M)) ||
        (has_keep && elements(keep) != M)) {
        return invalid("ln_projection: shapes do not match");
    }
    if (M == 0) return ok();
    if (!aligned16(x->data) || (n && (!aligned16(wT->data) || !aligned16(p->data))) ||
        (heads && !aligned16(wbT->data))) {
        return invalid("ln_projection: x, weights and p must be 16-byte aligned");
    }
    if (n == 0 && heads == 0) return ok();
    ProjArgs a{};
    a.x = f16p(x);
    a.scale = f32p(scale);
    a.offset = f32p(offset);
    a.wT = n ? f16p(wT) : nullptr;
    a.wbT = heads ? f16p(wbT) : nullptr;
    a.keep = has_keep ? f16p(keep) : nullptr;
    a.out = n ? static_cast<half_t*>(p->data) : nullptr;
    a.bias = heads ? static_cast<half_t*>(bias->data) : nullptr;
    a.M = (int)M;
    a.n = (int)n;
    a.heads = (int)heads;
    a.eps = eps;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (at == CLK_BF16) {
        return K == 64 ? run_proj<64, true, true>(a, s, "ln_projection")
                       : run_proj<128, true, true>(a, s, "ln_projection");
    }
    return K == 64 ? run_proj<64, true, false>(a, s, "ln_projection")
                   : run_proj<128, true, false>(a, s, "ln_projection");
}

extern "C" int clk_output_projection(clk_stream stream, const clk_buffer* o, const clk_buffer* wT,
                                     const clk_buffer* b, const clk_buffer* residual,
                                     const clk_buffer* keep, const clk_buffer* out, int32_t has_residual,
                                     int32_t has_keep) {
    const clk_buffer* bufs[] = {o, wT, b, residual, keep, out};
    const int at = act_type(o);
    const int types[] = {at, CLK_F16, CLK_F16, opt_act_type(residual, has_residual, at), CLK_F16, at};
    if (int st = check_types("output_projection", bufs, types, 6)) return st;
    if (o->rank != 2 || wT->rank != 2 || wT->dims[1] != o->dims[1]) {
        return invalid("output_projection: o must be [M,K] and wT [N,K]");
    }
    const int64_t M = o->dims[0], K = o->dims[1], N = wT->dims[0];
    if (!fused_width(K) || !fused_width(N)) return invalid("output_projection: K and N must be 64 or 128");
    if (elements(b) != N || elements(out) != M * N || (has_residual && elements(residual) != M * N) ||
        (has_keep && elements(keep) != M)) {
        return invalid("output_projection: shapes do not match");
    }
    if (M == 0) return ok();
    if (!aligned16(o->data) || !aligned16(wT->data) || !aligned16(out->data) ||
        (has_residual && !aligned16(residual->data))) {
        return invalid("output_projection: o, wT, residual and out must be 16-byte aligned");
    }
    ProjArgs a{};
    a.x = f16p(o);
    a.wT = f16p(wT);
    a.b = f16p(b);
    a.residual = has_residual ? f16p(residual) : nullptr;
    a.keep = has_keep ? f16p(keep) : nullptr;
    a.out = static_cast<half_t*>(out->data);
    a.M = (int)M;
    a.n = (int)N;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
#define CLK_OUTPROJ(K_, N_)                                                                            \
    if (K == K_ && N == N_) {                                                                          \
        if (at == CLK_BF16) {                                                                          \
            return has_residual ? run_outproj<K_, N_, true, true>(a, s)                                \
                                : run_outproj<K_, N_, false, true>(a, s);                              \
        }                                                                                              \
        return has_residual ? run_outproj<K_, N_, true, false>(a, s)                                   \
                            : run_outproj<K_, N_, false, false>(a, s);                                 \
    }
    CLK_OUTPROJ(64, 64) CLK_OUTPROJ(64, 128) CLK_OUTPROJ(128, 64) CLK_OUTPROJ(128, 128)
#undef CLK_OUTPROJ
    return invalid("output_projection: K and N must be 64 or 128");
}

template <bool ADD, bool BF>
static int run_transition_rows(const TransArgs& a, hipStream_t s) {
    const size_t lds = trans_rows_lds_bytes(64, a.H);
    const int64_t groups = ((a.M + kTransRowsTile - 1) / kTransRowsTile + kTransRowsThreads / kWave - 1) /
                           (kTransRowsThreads / kWave);
    const dim3 grid(persistent_grid(groups, lds, 1));
    if (int st = launch_fused("transition", transition_rows_kernel<ADD, BF>, grid, lds, s, &a, 0)) return st;
    stage_mark(s, 0);
    hipLaunchKernelGGL((transition_rows_kernel<ADD, BF>), grid, dim3(kTransRowsThreads), lds, s, a);
    stage_mark(s, 1);
    return launch_status("transition");
}

template <int C, bool ADD, bool BF>
static int run_transition(const TransArgs& a, hipStream_t s) {
    const int limit = fused_lds_limit();
    // C = 64: both weights resident in LDS (at most 66 KB at H = 4C); wider: the row tile, one
    // weight chunk, the LayerNorm parameters and the biases
    using T = TransTile<C>;
    constexpr int kTR = trans_rows<C>();
    const size_t lds = C == 64 ? trans_rows_lds_bytes(64, a.H)
                               : (size_t)kTR * C * 2 + (size_t)(T::kW1 + T::kW2) * 2 + (size_t)(3 * C + a.H) * 4;
    if (limit > 0 && lds > (size_t)limit) {
        return invalid("transition: needs " + std::to_string(lds / 1024) + " KB shared, device allows " +
                       std::to_string(limit / 1024) + " KB");
    }
    if constexpr (C == 64) {
        return run_transition_rows<ADD, BF>(a, s);
    } else {
        constexpr int TH = trans_threads(C);
        const int64_t tiles = (a.M + kTR - 1) / kTR;
        const dim3 grid(persistent_grid(tiles, lds, 1));
        if (int st = launch_fused("transition", transition_kernel<C, ADD, TH, BF>, grid, lds, s, &a, 0)) return st;
        stage_mark(s, 0);
        hipLaunchKernelGGL((transition_kernel<C, ADD, TH, BF>), grid, dim3(TH), lds, s, a);
        stage_mark(s, 1);
        return launch_status("transition");
    }
}

extern "C" int clk_transition(clk_stream stream, const clk_buffer* x, const clk_buffer* scale,
                              const clk_buffer* offset, const clk_buffer* w1T, const clk_buffer* b1,
                              const clk_buffer* w2T, const clk_buffer* b2, const clk_buffer* keep,
                              const clk_buffer* out, float eps, int32_t add_input, int32_t has_keep) {
    const clk_buffer* bufs[] = {x, scale, offset, w1T, b1, w2T, b2, keep, out};
    const int at = act_type(x);
    const int types[] = {at, CLK_F32, CLK_F32, CLK_F16, CLK_F16, CLK_F16, CLK_F16, CLK_F16, at};
    if (int st = check_types("transition", bufs, types, 9)) return st;
    if (x->rank != 2 || w1T->rank != 2 || w1T->dims[1] != x->dims[1]) {
        return invalid("transition: x must be [M,C] and w1T [H,C]");
    }
    const int64_t M = x->dims[0], C = x->dims[1], H = w1T->dims[0];
    if (!msa_width(C) || (H != 2 * C && H != 4 * C)) {
        return invalid("transition: C must be 64, 128 or 256, H 2C or 4C");
    }
    if (elements(scale) != C || elements(offset) != C || elements(b1) != H || elements(w2T) != H * C ||
        elements(b2) != C || elements(out) != M * C || (has_keep && elements(keep) != M)) {
        return invalid("transition: shapes do not match");
    }
    if (M == 0) return ok();
    if (!aligned16(x->data) || !aligned16(w1T->data) || !aligned16(w2T->data) || !aligned16(out->data)) {
        return invalid("transition: x, weights and out must be 16-byte aligned");
    }
    TransArgs a{f16p(x), f32p(scale), f32p(offset), f16p(w1T), f16p(b1), f16p(w2T), f16p(b2),
                has_keep ? f16p(keep) : nullptr, static_cast<half_t*>(out->data), (int)M, (int)H, eps};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (at == CLK_BF16) {
        if (C == 64) return add_input ? run_transition<64, true, true>(a, s) : run_transition<64, false, true>(a, s);
        if (C == 128) return add_input ? run_transition<128, true, true>(a, s) : run_transition<128, false, true>(a, s);
        return add_input ? run_transition<256, true, true>(a, s) : run_transition<256, false, true>(a, s);
    }
    if (C == 64) return add_input ? run_transition<64, true, false>(a, s) : run_transition<64, false, false>(a, s);
    if (C == 128) return add_input ? run_transition<128, true, false>(a, s) : run_transition<128, false, false>(a, s);
    return add_input ? run_transition<256, true, false>(a, s) : run_transition<256, false, false>(a, s);
}
