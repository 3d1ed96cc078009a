// The reference's unfused pair-stack ops for gfx950 (CDNA4): LayerNorm and the gated dual
// projection (reference cuda/volta_ops.cu:27-269, handlers VoltaLayerNorm and VoltaGdp).
//
//   layer_norm       out = fp16((x - mean) rstd scale + offset) over the last axis, with the
//                    reference's one-pass fp32 statistics: var = max(E[x^2] - mean^2, 0),
//                    rstd = rsqrt(var + eps) (volta_ops.cu:27-57). A row is split over C/8 lanes
//                    holding one 16-byte chunk each when C % 8 == 0, else over a whole wave.
//   gated_dual_proj  out[m, n] = fp16(mask[m] (x@wp + bp)[m, n] act((x@wg + bg)[m, n])) with
//                    wp, wg row-major [K, N] and act sigmoid or swish (volta_ops.cu:97-269,
//                    volta_gdp.h:10-35). A workgroup computes a 64 x 64 output tile as
//                    out^T = W^T X^T on MFMA: K steps of 32 stage x [64 x 32] and both weight
//                    tiles [32 x 64] row-major in LDS, and the W^T operand is read with the
//                    gfx950 transpose load straight from the row-major weight tile.
#include "clk_common.h"

namespace clk {

// ---- layer_norm ---------------------------------------------------------------------------

struct LnArgs {
    const half_t* x;
    const float* scale;
    const float* offset;
    half_t* out;
    int64_t M;
    int C;
    float eps;
};

// C % 8 == 0: TPR = C / 8 lanes per row (a power of two up to 64), one 16-byte chunk each
template <int TPR>
__global__ __launch_bounds__(256) void layer_norm_vec_kernel(LnArgs a) {
    constexpr int RPW = kWave / TPR;  // rows per wave
    const int lane = threadIdx.x & (kWave - 1), part = lane % TPR, sub = lane / TPR;
    const int64_t waves = (int64_t)gridDim.x * (blockDim.x / kWave);
    const int64_t wave0 = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
    const int col = 8 * part;
    float sc[8], of[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        sc[e] = a.scale[col + e];
        of[e] = a.offset[col + e];
    }
    for (int64_t r0 = wave0 * RPW; r0 < a.M; r0 += waves * RPW) {
        const int64_t row = r0 + sub;
        const bool in = row < a.M;
        const half8 v = in ? *reinterpret_cast<const half8*>(a.x + row * a.C + col) : half8{};
        float s = 0.f, q = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float f = (float)v[e];
            s += f;
            q += f * f;
        }
#pragma unroll
        for (int o = 1; o < TPR; o <<= 1) {
            s += __shfl_xor(s, o);
            q += __shfl_xor(q, o);
        }
        const float inv = 1.f / (float)a.C;
        const float mean = s * inv;
        const float var = fmaxf(q * inv - mean * mean, 0.f);
        const float rstd = __builtin_amdgcn_rsqf(var + a.eps);
        if (in) {
            half8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (half_t)(((float)v[e] - mean) * rstd * sc[e] + of[e]);
            *reinterpret_cast<half8*>(a.out + row * a.C + col) = o;
        }
    }
}

// any C: a wave per row, lanes strided over it
__global__ __launch_bounds__(256) void layer_norm_any_kernel(LnArgs a) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t waves = (int64_t)gridDim.x * (blockDim.x / kWave);
    for (int64_t row = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave; row < a.M;
         row += waves) {
        const half_t* xr = a.x + row * a.C;
        float s = 0.f, q = 0.f;
        for (int c = lane; c < a.C; c += kWave) {
            const float f = (float)xr[c];
            s += f;
            q += f * f;
        }
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            s += __shfl_xor(s, o);
            q += __shfl_xor(q, o);
        }
        const float inv = 1.f / (float)a.C;
        const float mean = s * inv;
        const float var = fmaxf(q * inv - mean * mean, 0.f);
        const float rstd = __builtin_amdgcn_rsqf(var + a.eps);
        for (int c = lane; c < a.C; c += kWave) {
            a.out[row * a.C + c] = (half_t)(((float)xr[c] - mean) * rstd * a.scale[c] + a.offset[c]);
        }
    }
}

// ---- gated_dual_proj ----------------------------------------------------------------------

struct GdpArgs {
    const half_t *x, *wp, *bp, *wg, *bg, *mask;
    half_t* out;
    int M, K, N;
    bool xvec, wvec;  // 16-byte loads of x rows / weight rows are aligned
};

constexpr int kGdpBM = 64, kGdpBN = 64, kGdpBK = 32;
constexpr int kGdpXLd = kGdpBK + 8;  // x tile row stride (halfs)
constexpr int kGdpWLd = kGdpBN + 8;  // weight tile row stride (halfs)

template <bool SWISH>
__device__ __forceinline__ float gdp_act(float g) {
    const float s = sigmoid_fast(g);
    return SWISH ? g * s : s;
}

// 8 consecutive halfs of a row of length `len` starting at `col`, zero past `len`
__device__ __forceinline__ half8 load_row8(const half_t* row, int col, int len, bool vec) {
    if (vec && col + 8 <= len) return *reinterpret_cast<const half8*>(row + col);
    half8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = col + e < len ? row[col + e] : (half_t)0.f;
    return v;
}

// Four waves; wave w owns output columns n0 + 16 w .. +15 for all 64 rows (four 16-row blocks).
// A row r of the W^T block is n = n0 + 16 w + r; B column of row block rb is m = m0 + 16 rb + col.
template <bool SWISH>
__global__ __launch_bounds__(256) void gdp_kernel(GdpArgs a) {
    __shared__ __attribute__((aligned(16))) half_t Xs[kGdpBM * kGdpXLd];
    __shared__ __attribute__((aligned(16))) half_t Ps[kGdpBK * kGdpWLd];
    __shared__ __attribute__((aligned(16))) half_t Gs[kGdpBK * kGdpWLd];
    const int m0 = blockIdx.x * kGdpBM, n0 = blockIdx.y * kGdpBN;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int r16 = lane & 15, g = lane >> 4;

    float4v ap[4], ag[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        ap[rb] = float4v{0.f, 0.f, 0.f, 0.f};
        ag[rb] = float4v{0.f, 0.f, 0.f, 0.f};
    }
    for (int k0 = 0; k0 < a.K; k0 += kGdpBK) {
        __syncthreads();
        {   // x tile: 64 rows x 4 chunks; weight tiles: 32 rows x 8 chunks each
            const int xr = tid >> 2, xc = (tid & 3) * 8;
            const int gm = m0 + xr;
            const half8 xv = gm < a.M ? load_row8(a.x + (int64_t)gm * a.K, k0 + xc, a.K, a.xvec) : half8{};
            *reinterpret_cast<half8*>(&Xs[xr * kGdpXLd + xc]) = xv;
            const int wr = tid >> 3, wc = (tid & 7) * 8;
            const int gk = k0 + wr;
            const bool kin = gk < a.K;
            const half8 pv = kin ? load_row8(a.wp + (int64_t)gk * a.N, n0 + wc, a.N, a.wvec) : half8{};
            const half8 gv = kin ? load_row8(a.wg + (int64_t)gk * a.N, n0 + wc, a.N, a.wvec) : half8{};
            *reinterpret_cast<half8*>(&Ps[wr * kGdpWLd + wc]) = pv;
            *reinterpret_cast<half8*>(&Gs[wr * kGdpWLd + wc]) = gv;
        }
        __syncthreads();
        // A = W^T (row n, k-slots 8 g + j) by transpose reads of the row-major [k][n] tiles
        const auto prow = [&](int r) { return Ps + r * kGdpWLd; };
        const auto grow = [&](int r) { return Gs + r * kGdpWLd; };
        const half8 wpa = lds_operand_tr(prow, g, r16, 16 * wave, 4);
        const half8 wga = lds_operand_tr(grow, g, r16, 16 * wave, 4);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const half8 xb = *reinterpret_cast<const half8*>(&Xs[(16 * rb + r16) * kGdpXLd + 8 * g]);
            ap[rb] = mfma16x16x32(wpa, xb, ap[rb]);
            ag[rb] = mfma16x16x32(wga, xb, ag[rb]);
        }
    }
    // lane holds out[m][n .. n+3]: m = m0 + 16 rb + r16, n = n0 + 16 wave + 4 g
    const int n = n0 + 16 * wave + 4 * g;
    if (n >= a.N) return;  // N % 8 == 0, so these 4 columns are all in or all out
    float bpv[4], bgv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        bpv[i] = (float)a.bp[n + i];
        bgv[i] = (float)a.bg[n + i];
    }
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        const int m = m0 + 16 * rb + r16;
        if (m >= a.M) continue;
        const float mv = (float)a.mask[m];
        half4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = ap[rb][i] + bpv[i];
            o[i] = (half_t)(mv * p * gdp_act<SWISH>(ag[rb][i] + bgv[i]));
        }
        *reinterpret_cast<half4*>(a.out + (int64_t)m * a.N + n) = o;
    }
}

// The same op as a persistent, straight-line kernel for K in {64, 128} and N in {64, 128, 256}:
// eight waves, wave w owning column pair w / SPLIT (32 outputs) and RBW of a 64-row tile's four
// row blocks. The wave's A operands (W^T rows of its pair, both matrices) are gathered into
// registers once; per tile only x passes through LDS, as B-operand fragments. The next tile's rows
// and mask are fetched before this tile's stores and consumed after them in the same iteration,
// so no wait for a load covers a store (vmcnt counts both in issue order). Results are 16-byte
// buffer stores through a per-tile descriptor, so rows past M are dropped without a branch.
// workgroups per CU the fast kernel is compiled for: its registers allow two at K = 64, one at 128
constexpr int gdp_per_cu(int K) { return K == 64 ? 2 : 1; }

template <int K, int N, bool SWISH>
__global__ __launch_bounds__(512, 2 * gdp_per_cu(K)) void gdp_fast_kernel(GdpArgs a) {
    constexpr int TH = 512, KS = K / 32, TW = TH / kWave, KC = K / 8;
    constexpr int NPAIRS = N / 32, SPLIT = TW / NPAIRS, RBW = 4 / SPLIT;
    static_assert(TW % NPAIRS == 0 && 4 % SPLIT == 0, "whole row blocks per wave");
    constexpr int XCPT = kGdpBM * KC / TH;  // 16-byte chunks of the x tile per thread
    static_assert(XCPT >= 1 && kGdpBM * KC % TH == 0, "whole chunks per thread");
    using u32x4 = unsigned int __attribute__((ext_vector_type(4)));
    // block rb, step ks, lane (row 16 rb + lane % 16, k-slots 32 ks + 8 (lane / 16) ..)
    __shared__ __attribute__((aligned(16))) half_t Xf[kGdpBM * K];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int r16 = lane & 15, g = lane >> 4;
    const int cp = wave / SPLIT, rb0 = (wave % SPLIT) * RBW;
    const int col = 32 * cp + 8 * g;
    const int tiles = (a.M + kGdpBM - 1) / kGdpBM;
    const int G = gridDim.x;

    // A-operand row r16 of block hb: output column 32 cp + 8 (r16 / 4) + 4 hb + r16 % 4, so the
    // accumulators give lane group g the 8 consecutive columns col .. col + 7
    half8 wpa[2][KS], wga[2][KS];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
        const int n = 32 * cp + 8 * (r16 >> 2) + 4 * hb + (r16 & 3);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int64_t k = 32 * ks + 8 * g + e;
                wpa[hb][ks][e] = a.wp[k * N + n];
                wga[hb][ks][e] = a.wg[k * N + n];
            }
    }
    float bpv[8], bgv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        bpv[j] = (float)a.bp[col + j];
        bgv[j] = (float)a.bg[col + j];
    }

    // tile t's x chunks (rows past M repeat row M - 1; their results are dropped) and the mask of
    // the lane's output row in each of its row blocks
    half8 xv[XCPT];
    half_t mraw[RBW];
    const auto fetch = [&](int t) {
        const int m0 = t * kGdpBM;
#pragma unroll
        for (int j = 0; j < XCPT; ++j) {
            const int q = threadIdx.x + TH * j, row = q / KC, c = q % KC;
            xv[j] = *reinterpret_cast<const half8*>(a.x + (int64_t)min(m0 + row, a.M - 1) * K + 8 * c);
        }
#pragma unroll
        for (int i = 0; i < RBW; ++i) mraw[i] = a.mask[min(m0 + 16 * (rb0 + i) + r16, a.M - 1)];
    };
    float mv[RBW];
    const auto prepare = [&]() {
        __syncthreads();  // the previous tile's operand reads are done
#pragma unroll
        for (int j = 0; j < XCPT; ++j) {
            const int q = threadIdx.x + TH * j, row = q / KC, c = q % KC;
            const int l = (row & 15) + 16 * (c & 3);
            *reinterpret_cast<half8*>(&Xf[(((row >> 4) * KS + (c >> 2)) * kWave + l) * 8]) = xv[j];
        }
#pragma unroll
        for (int i = 0; i < RBW; ++i) mv[i] = pin_f32((float)mraw[i]);  // here, not after the next fetch
        __syncthreads();
    };
    const auto gemm_store = [&](int t) {
        const int m0 = t * kGdpBM;
        const uint32_t rows = (uint32_t)min(kGdpBM, a.M - m0);
        const auto ro = __builtin_amdgcn_make_buffer_rsrc(a.out + (int64_t)m0 * N, 0, rows * N * 2u, 0x00020000);
#pragma unroll
        for (int i = 0; i < RBW; ++i) {
            const int rb = rb0 + i;
            float4v ap[2], ag[2];
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                ap[hb] = float4v{0.f, 0.f, 0.f, 0.f};
                ag[hb] = float4v{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const half8 xb = *reinterpret_cast<const half8*>(&Xf[((rb * KS + ks) * kWave + lane) * 8]);
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) {
                    ap[hb] = mfma16x16x32(wpa[hb][ks], xb, ap[hb]);
                    ag[hb] = mfma16x16x32(wga[hb][ks], xb, ag[hb]);
                }
            }
            half8 o;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = ap[j >> 2][j & 3] + bpv[j];
                o[j] = (half_t)(mv[i] * p * gdp_act<SWISH>(ag[j >> 2][j & 3] + bgv[j]));
            }
            const uint32_t off = (uint32_t)((16 * rb + r16) * N + col) * 2u;
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), ro, off, 0, 0);
        }
    };

    int t = blockIdx.x;
    if (t >= tiles) return;
    fetch(t);
    prepare();
    for (;;) {
        const int nt = t + G;
        fetch(min(nt, tiles - 1));
        gemm_store(t);
        if (nt >= tiles) break;
        t = nt;
        prepare();
    }
}

}  // namespace clk

using namespace clk;

extern "C" int clk_layer_norm(clk_stream stream, const clk_buffer* x, const clk_buffer* scale,
                              const clk_buffer* offset, const clk_buffer* out, float eps) {
    const clk_buffer* bufs[] = {x, scale, offset, out};
    const int types[] = {CLK_F16, CLK_F32, CLK_F32, CLK_F16};
    if (int st = check_types("layer_norm", bufs, types, 4)) return st;
    if (x->rank != 2) return invalid("x must be [M,C]");
    const int64_t M = x->dims[0], C = x->dims[1];
    if (elements(scale) != C || elements(offset) != C || !same_shape(out, x)) {
        return invalid("layer_norm: scale and offset must be [C], out like x");
    }
    if (M == 0 || C == 0) return ok();
    if (C > INT32_MAX) return invalid("layer_norm: C too large");
    LnArgs a{static_cast<const half_t*>(x->data), static_cast<const float*>(scale->data),
             static_cast<const float*>(offset->data), static_cast<half_t*>(out->data), M, (int)C, eps};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool vec = C % 8 == 0 && C / 8 <= kWave && ((C / 8) & (C / 8 - 1)) == 0 &&
                     aligned16(x->data) && aligned16(out->data);
    stage_mark(s, 0);
    if (vec) {
        const int tpr = (int)(C / 8);
        const int64_t rows_per_block = 256 / tpr;
        const unsigned blocks = (unsigned)std::min<int64_t>((M + rows_per_block - 1) / rows_per_block, 65535);
#define CLK_LN(T_) if (tpr == T_) hipLaunchKernelGGL(layer_norm_vec_kernel<T_>, dim3(blocks), dim3(256), 0, s, a);
        CLK_LN(1) CLK_LN(2) CLK_LN(4) CLK_LN(8) CLK_LN(16) CLK_LN(32) CLK_LN(64)
#undef CLK_LN
    } else {
        const unsigned blocks = (unsigned)std::min<int64_t>((M + 3) / 4, 65535);
        hipLaunchKernelGGL(layer_norm_any_kernel, dim3(blocks), dim3(256), 0, s, a);
    }
    stage_mark(s, 1);
    return launch_status("layer_norm");
}

extern "C" int clk_gated_dual_proj(clk_stream stream, int32_t device, const clk_buffer* x,
                                   const clk_buffer* wp, const clk_buffer* bp, const clk_buffer* wg,
                                   const clk_buffer* bg, const clk_buffer* mask, const clk_buffer* out,
                                   int64_t activation) {
    (void)device;
    const clk_buffer* bufs[] = {x, wp, bp, wg, bg, mask, out};
    const int types[] = {CLK_F16, CLK_F16, CLK_F16, CLK_F16, CLK_F16, CLK_F16, CLK_F16};
    if (int st = check_types("gated_dual_proj", bufs, types, 7)) return st;
    if (x->rank != 2) return invalid("x must be [M,K]");
    const int64_t M = x->dims[0], K = x->dims[1];
    if (wp->rank != 2 || wp->dims[0] != K || !same_shape(wg, wp)) {
        return invalid("gdp: wp and wg must be [K,N]");
    }
    const int64_t N = wp->dims[1];
    if (N % 8) return invalid("gdp: N must be a multiple of 8");
    if (activation != 0 && activation != 1) {
        return invalid("gdp: activation is 0 (sigmoid) or 1 (swish), got " + std::to_string(activation));
    }
    if (elements(bp) != N || elements(bg) != N || elements(mask) != M || out->rank != 2 ||
        out->dims[0] != M || out->dims[1] != N) {
        return invalid("gdp: bp, bg must be [N], mask [M], out [M,N]");
    }
    if (M == 0 || N == 0) return ok();
    if (M > INT32_MAX || K > INT32_MAX || N > INT32_MAX) return invalid("gdp: too large");
    if (!aligned16(out->data)) return invalid("gdp: out must be 16-byte aligned");
    GdpArgs a{static_cast<const half_t*>(x->data), static_cast<const half_t*>(wp->data),
              static_cast<const half_t*>(bp->data), static_cast<const half_t*>(wg->data),
              static_cast<const half_t*>(bg->data), static_cast<const half_t*>(mask->data),
              static_cast<half_t*>(out->data), (int)M, (int)K, (int)N,
              K % 8 == 0 && aligned16(x->data), aligned16(wp->data) && aligned16(wg->data)};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if ((K == 64 || K == 128) && (N == 64 || N == 128 || N == 256) && aligned16(x->data)) {
        // persistent: as many workgroups as the registers it is compiled for let a CU hold
        int dev = 0, cus = 256;
        if (hipGetDevice(&dev) == hipSuccess) {
            int v = 0;
            if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
        }
        const int64_t tiles = (M + kGdpBM - 1) / kGdpBM;
        const dim3 pgrid((unsigned)std::min<int64_t>(tiles, (int64_t)gdp_per_cu((int)K) * cus));
#define CLK_GDP_FAST(K_, N_)                                                                           \
        if (K == K_ && N == N_) {                                                                      \
            stage_mark(s, 0);                                                                          \
            if (activation == 0) hipLaunchKernelGGL((gdp_fast_kernel<K_, N_, false>), pgrid, dim3(512), 0, s, a); \
            else hipLaunchKernelGGL((gdp_fast_kernel<K_, N_, true>), pgrid, dim3(512), 0, s, a);     \
            stage_mark(s, 1);                                                                          \
            return launch_status("gated_dual_proj");                                                   \
        }
        CLK_GDP_FAST(64, 64) CLK_GDP_FAST(64, 128) CLK_GDP_FAST(64, 256)
        CLK_GDP_FAST(128, 64) CLK_GDP_FAST(128, 128) CLK_GDP_FAST(128, 256)
#undef CLK_GDP_FAST
    }
    const dim3 grid((unsigned)((M + kGdpBM - 1) / kGdpBM), (unsigned)((N + kGdpBN - 1) / kGdpBN));
    if (grid.y > 65535) return invalid("gdp: N too large");
    stage_mark(s, 0);
    if (activation == 0) {
        hipLaunchKernelGGL(gdp_kernel<false>, grid, dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL(gdp_kernel<true>, grid, dim3(256), 0, s, a);
    }
    stage_mark(s, 1);
    return launch_status("gated_dual_proj");
}
