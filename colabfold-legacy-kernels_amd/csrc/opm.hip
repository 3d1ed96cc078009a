// The outer product mean kernels for gfx950 (CDNA4): opm_update and opm_outer (reference
// cuda/volta_ops.cu:643-792, handlers cuda/volta_fused_ffi.h:261-335, 420-440).
//
//   opm_update  out[b, d, f] = fp16((sum_k lhs[b, k] t[k, d, f] + bias[f]) / (eps + norm[b, d])
//               [+ residual[b, d, f]]), fp32 accumulation. A GEMM over N = D F columns: a
//               workgroup computes a 64 (b) x 64 (n) tile as out^T = t^T lhs^T on MFMA, K steps of
//               32 staging lhs and t row-major in LDS; the t^T operand is read with the gfx950
//               transpose load.
//   opm_outer   out[b, d, f] = fp16(sum_c sum_e fp16(sum_a left[a, b, c] right[a, d, e])
//               w[c E + e, f]) over the 16 rows a, E = 32, wT [F, C E]. A workgroup owns 16 rows b
//               and 4 columns d, one wave per d. For each channel c the wave forms
//               G^T[e, b] = sum_a right[a, d, e] left[a, b, c] with a 16x16x16 MFMA whose A rows
//               are e in pair order, so that the accumulator, rounded to fp16, is already the B
//               operand (k-slots e) of out^T[f, b] += W_c^T G_c^T, a 16x16x32 MFMA against the
//               channel's weight rows staged in LDS. The [B, C E, D] product is never formed.
#include "clk_common.h"

namespace clk {

__device__ __forceinline__ float4v mfma16x16x16(half4 a, half4 b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// ---- opm_update ---------------------------------------------------------------------------

struct OpmUpdateArgs {
    const half_t *lhs, *t, *residual;  // lhs [B, K], t [K, D F], residual [B, D F] or null
    const float *bias, *norm;          // bias [F], norm [B, D]
    half_t* out;                       // [B, D F]
    int B, K, D, F;
    float eps;
};

constexpr int kUpBM = 64, kUpBN = 64;
constexpr int kUpTLd = kUpBN + 8;

// Four waves: waves 2 p and 2 p + 1 own the column pair n0 + 32 p .. +31, rows 0-31 and 32-63 of
// the tile. The A rows of column block hb are n0 + 32 p + 8 (r / 4) + 4 hb + r % 4, so the
// accumulators give a lane 8 consecutive columns of one row (16-byte stores). Work items are
// column-tile-major, with the row tiles of one column tile consecutive on one XCD (xcd_item):
// they share the t tile, which HBM then serves once. The next K step's chunks are loaded (from
// clamped addresses, unconditionally) before this step's products, and the epilogue's residual,
// norm and bias before the K loop, so no wait covers a store. A K step is BK deep (128, 64 or 32,
// the largest that divides K), so each barrier pair covers BK / 32 products per column block.
template <int BK>
__global__ __launch_bounds__(256) void opm_update_kernel(OpmUpdateArgs a) {
    constexpr int kUpXLd = BK + 8, XCPT = BK / 32, TCPT = BK / 32;  // 16-byte chunks per thread
    __shared__ __attribute__((aligned(16))) half_t Xs[kUpBM * kUpXLd];
    __shared__ __attribute__((aligned(16))) half_t Ts[BK * kUpTLd];
    const int N = a.D * a.F;
    const int mtiles = (a.B + kUpBM - 1) / kUpBM;
    const int item = xcd_item(blockIdx.x, gridDim.x);
    const int m0 = (item % mtiles) * kUpBM, n0 = (item / mtiles) * kUpBN;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int r16 = lane & 15, g = lane >> 4;
    const int p = wave >> 1, rh = wave & 1;

    // epilogue operands: lane holds out[b][n .. n+7], b = m0 + 32 rh + 16 i + r16, one d (F >= 16)
    const int n = n0 + 32 * p + 8 * g;
    const bool nin = n < N;  // N is a multiple of 16: 8 columns are wholly in or out
    const int nc = min(n, N - 8), d = nc / a.F, f = nc - d * a.F;
    float bv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) bv[j] = a.bias[f + j];
    float den[2];
    half8 res[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int b = min(m0 + 32 * rh + 16 * i + r16, a.B - 1);
        den[i] = a.eps + a.norm[(int64_t)b * a.D + d];
        res[i] = half8{};
        if (a.residual != nullptr)  // may alias out: read before any write
            res[i] = *reinterpret_cast<const half8*>(a.residual + (int64_t)b * N + nc);
    }

    float4v acc[2][2];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[hb][i] = float4v{0.f, 0.f, 0.f, 0.f};
    // this thread's chunks of each K step: x chunk (row xr, columns xc + 32 u), t chunk (row tr +
    // 32 u, columns tc); rows past B and columns past N repeat the last ones (their results are not
    // stored); K is a multiple of BK
    const int xr = tid >> 2, xc = (tid & 3) * 8, tr = tid >> 3, tc = (tid & 7) * 8;
    const half_t* xrow = a.lhs + (int64_t)min(m0 + xr, a.B - 1) * a.K + xc;
    const half_t* tcol = a.t + (int64_t)tr * N + min(n0 + tc, N - 8);
    half8 xv[XCPT], tv[TCPT];
    const auto fetch = [&](int k0) {
#pragma unroll
        for (int u = 0; u < XCPT; ++u) xv[u] = *reinterpret_cast<const half8*>(xrow + k0 + 32 * u);
#pragma unroll
        for (int u = 0; u < TCPT; ++u) tv[u] = *reinterpret_cast<const half8*>(tcol + (int64_t)(k0 + 32 * u) * N);
    };
    fetch(0);
    for (int k0 = 0; k0 < a.K; k0 += BK) {
        __syncthreads();  // the previous step's operand reads are done
#pragma unroll
        for (int u = 0; u < XCPT; ++u) *reinterpret_cast<half8*>(&Xs[xr * kUpXLd + xc + 32 * u]) = xv[u];
#pragma unroll
        for (int u = 0; u < TCPT; ++u) *reinterpret_cast<half8*>(&Ts[(tr + 32 * u) * kUpTLd + tc]) = tv[u];
        __syncthreads();
        fetch(min(k0 + BK, a.K - BK));
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            half8 top[2];
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
                top[hb] = lds_operand_tr([&](int r) { return Ts + (32 * ks + r) * kUpTLd; }, g, r16, 32 * p + 4 * hb, 8);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const half8 xb =
                    *reinterpret_cast<const half8*>(&Xs[(32 * rh + 16 * i + r16) * kUpXLd + 32 * ks + 8 * g]);
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) acc[hb][i] = mfma16x16x32(top[hb], xb, acc[hb][i]);
            }
        }
    }
    if (!nin) return;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int b = m0 + 32 * rh + 16 * i + r16;
        if (b >= a.B) continue;
        half8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = (half_t)((acc[j >> 2][i][j & 3] + bv[j]) / den[i] + (float)res[i][j]);
        *reinterpret_cast<half8*>(a.out + (int64_t)b * N + n) = h;
    }
}

// ---- opm_outer ----------------------------------------------------------------------------

constexpr int kOpmRows = 16, kOpmE = 32, kOpmB = 16, kOpmD = 4, kOpmChunk = 16;
constexpr int kLtLd = kOpmRows + 4;  // Lt[c][b][a] row stride (halfs), 8-byte aligned rows
// Lt channel stride (halfs): 4 halfs past the 16 rows, so that channels 8 apart (the two 8-channel
// halves a staging store instruction writes) fall on different LDS banks
constexpr int kLtCh = kOpmB * kLtLd + 4;

struct OpmOuterArgs {
    const half_t *left, *right, *wT;  // left [16, B, C], right [16, D, 32], wT [F, 32 C]
    half_t* out;                      // [B, D, F]
    int B, C, D;
};

// e of A row r in e block eb of the first product: lane group g of its accumulator then holds
// e = 8 g + 4 eb + i, i.e. the k-slots 8 g .. 8 g + 7 of the second product's B operand
__device__ __forceinline__ int opm_e(int eb, int r) { return 8 * (r >> 2) + 4 * eb + (r & 3); }

// DPW columns d per wave (1, or 2 where D % 8 == 0): the channel's staged weights and left values
// then serve DPW times as many outputs per barrier.
template <int F, int DPW>
__global__ __launch_bounds__(256) void opm_outer_kernel(OpmOuterArgs a) {
    constexpr int FB = F / 16;
    constexpr int kWLd = kOpmE + 8;  // Ws row stride (halfs)
    __shared__ __attribute__((aligned(16))) half_t Lt[kOpmChunk * kLtCh];
    __shared__ __attribute__((aligned(16))) half_t Ws[2][2][F * kWLd];  // [buffer][channel of the pair]
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int r16 = lane & 15, g = lane >> 4;
    const int b0 = blockIdx.x * kOpmB, d0 = blockIdx.y * kOpmD * DPW + wave;  // d = d0 + kOpmD j

    // right[:, d] as the A operand of the first product: row r of e block eb is e = opm_e(eb, r),
    // k-slots a = 4 g .. 4 g + 3
    half4 ra[DPW][2];
#pragma unroll
    for (int dj = 0; dj < DPW; ++dj)
#pragma unroll
        for (int eb = 0; eb < 2; ++eb)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                ra[dj][eb][j] = a.right[((int64_t)(4 * g + j) * a.D + d0 + kOpmD * dj) * kOpmE + opm_e(eb, r16)];

    // The weight rows of a pair of channels c, c + 1 (Ws[.][h][f][e] = wT[f][32 (c + h) + e]), a
    // step per barrier, and the left values of a chunk of 16 channels (Lt[c][b][a] =
    // left[a][b0 + b][c0 + c]) pass through registers one step (weights) or one chunk (left)
    // before they are stored to LDS, so their loads are in flight during a step's products
    // instead of being waited for at once.
    constexpr int WCH = F * (kOpmE / 8);                        // 16-byte weight chunks per channel
    constexpr int WCPT = (WCH + 255) / 256;                     // per thread
    half8 wreg[2][WCPT], lreg[2];
    // channels c and c + 1 (a pair: C is a multiple of 16)
    const auto fetch_w = [&](int c) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int u = 0; u < WCPT; ++u) {
                const int i = min(tid + 256 * u, WCH - 1);
                const int f = i / (kOpmE / 8), e8 = (i % (kOpmE / 8)) * 8;
                wreg[h][u] = *reinterpret_cast<const half8*>(a.wT + (int64_t)f * a.C * kOpmE + (c + h) * kOpmE + e8);
            }
    };
    const auto store_w = [&](int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int u = 0; u < WCPT; ++u) {
                const int i = tid + 256 * u;
                if (i < WCH) {
                    const int f = i / (kOpmE / 8), e8 = (i % (kOpmE / 8)) * 8;
                    *reinterpret_cast<half8*>(&Ws[buf][h][f * kWLd + e8]) = wreg[h][u];
                }
            }
    };
    // The first product's B operand gives lane (b, g) rows a = 4 g .. +3 of one channel and row b:
    // 8 bytes at Lt[c][b][4 g]. So a thread stages rows a = 2 lp and 2 lp + 1 of row b = lb for the
    // eight channels of half lv of the chunk (two 16-byte loads, consecutive lanes covering the two
    // halves of a 32-byte run of a row) and writes each channel's two values as one 4-byte store.
    // Rows b past B repeat the last row (their results are not stored).
    static_assert(kOpmRows / 2 * kOpmB * (kOpmChunk / 8) == 256, "one (row pair, row b, half) per thread");
    const int lv = tid & 1, lb = (tid >> 1) & (kOpmB - 1), lp = tid >> 5;
    const auto fetch_left = [&](int c0) {
        const half_t* src = a.left + ((int64_t)(2 * lp) * a.B + min(b0 + lb, a.B - 1)) * a.C + c0 + 8 * lv;
        lreg[0] = *reinterpret_cast<const half8*>(src);
        lreg[1] = *reinterpret_cast<const half8*>(src + (int64_t)a.B * a.C);
    };
    const auto store_left = [&]() {
        half_t* dst = &Lt[8 * lv * kLtCh + lb * kLtLd + 2 * lp];
#pragma unroll
        for (int j = 0; j < 8; ++j) *reinterpret_cast<half2v*>(dst + j * kLtCh) = half2v{lreg[0][j], lreg[1][j]};
    };

    float4v acc[DPW][FB];
#pragma unroll
    for (int dj = 0; dj < DPW; ++dj)
#pragma unroll
        for (int fb = 0; fb < FB; ++fb) acc[dj][fb] = float4v{0.f, 0.f, 0.f, 0.f};

    fetch_left(0);
    fetch_w(0);
    store_w(0);
    fetch_w(min(2, a.C - 2));
    for (int c = 0; c < a.C; c += 2) {
        const int cl = c % kOpmChunk, buf = (c >> 1) & 1;
        if (cl == 0) {
            __syncthreads();  // the previous chunk's Lt reads are done
            store_left();
            fetch_left(min(c + kOpmChunk, a.C - kOpmChunk));
        }
        __syncthreads();  // Lt of this chunk and Ws[buf] of this pair are staged; Ws[buf ^ 1] is free
        store_w(buf ^ 1);               // channels c + 2, c + 3, fetched a step ago
        fetch_w(min(c + 4, a.C - 2));   // channels c + 4, c + 5
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // G^T[e][b] for channel c + h: B operand L^T (lane column b, k-slots a = 4 g .. 4 g + 3)
            const half4 lbop = *reinterpret_cast<const half4*>(&Lt[(cl + h) * kLtCh + r16 * kLtLd + 4 * g]);
            half8 gop[DPW];
#pragma unroll
            for (int dj = 0; dj < DPW; ++dj)
#pragma unroll
                for (int eb = 0; eb < 2; ++eb) {
                    const float4v gt = mfma16x16x16(ra[dj][eb], lbop, float4v{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int i = 0; i < 4; ++i) gop[dj][4 * eb + i] = (half_t)gt[i];  // the f16 outer product
                }
            // out^T[f][b] += W^T G^T: A row r of f block fb is f = 16 fb + r, k-slots e = 8 g + j
#pragma unroll
            for (int fb = 0; fb < FB; ++fb) {
                const half8 w = *reinterpret_cast<const half8*>(&Ws[buf][h][(16 * fb + r16) * kWLd + 8 * g]);
#pragma unroll
                for (int dj = 0; dj < DPW; ++dj) acc[dj][fb] = mfma16x16x32(w, gop[dj], acc[dj][fb]);
            }
        }
    }
    // lane holds out[b][d][f .. f+3], b = b0 + r16, f = 16 fb + 4 g
    const int b = b0 + r16;
    if (b >= a.B) return;
#pragma unroll
    for (int dj = 0; dj < DPW; ++dj)
#pragma unroll
        for (int fb = 0; fb < FB; ++fb) {
            half4 h;
#pragma unroll
            for (int i = 0; i < 4; ++i) h[i] = (half_t)acc[dj][fb][i];
            *reinterpret_cast<half4*>(a.out + ((int64_t)b * a.D + d0 + kOpmD * dj) * F + 16 * fb + 4 * g) = h;
        }
}

static bool opm_width(int64_t f) { return f == 16 || f == 32 || f == 64 || f == 128; }

}  // namespace clk

using namespace clk;

extern "C" int clk_opm_update(clk_stream stream, const clk_buffer* lhs, const clk_buffer* t,
                              const clk_buffer* bias, const clk_buffer* norm,
                              const clk_buffer* residual, const clk_buffer* out, float eps,
                              int32_t has_residual) {
    const clk_buffer* bufs[] = {lhs, t, bias, norm, residual, out};
    const int types[] = {CLK_F16, CLK_F16, CLK_F32, CLK_F32, CLK_F16, CLK_F16};
    if (int st = check_types("opm_update", bufs, types, 6)) return st;
    if (lhs->rank != 2 || t->rank != 3 || t->dims[0] != lhs->dims[1]) {
        return invalid("opm_update: lhs must be [B,K] and t [K,D,F]");
    }
    const int64_t B = lhs->dims[0], K = lhs->dims[1], D = t->dims[1], F = t->dims[2];
    if (K % 32 || !opm_width(F) || D > 65535) {
        return invalid("opm_update: K must be a multiple of 32, F 16, 32, 64 or 128, D at most 65535");
    }
    if (elements(bias) != F || elements(norm) != B * D || elements(out) != B * D * F ||
        (has_residual && elements(residual) != B * D * F)) {
        return invalid("opm_update: shapes do not match");
    }
    if (B == 0 || D == 0) return ok();
    if (!aligned16(lhs->data) || !aligned16(t->data) || !aligned16(out->data) ||
        (has_residual && !aligned16(residual->data))) {
        return invalid("opm_update: lhs, t, residual and out must be 16-byte aligned");
    }
    if ((B + kUpBM - 1) / kUpBM > 65535 || K > INT32_MAX) return invalid("opm_update: too large");
    OpmUpdateArgs a{static_cast<const half_t*>(lhs->data), static_cast<const half_t*>(t->data),
                    has_residual ? static_cast<const half_t*>(residual->data) : nullptr,
                    static_cast<const float*>(bias->data), static_cast<const float*>(norm->data),
                    static_cast<half_t*>(out->data), (int)B, (int)K, (int)D, (int)F, eps};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t items = ((D * F + kUpBN - 1) / kUpBN) * ((B + kUpBM - 1) / kUpBM);
    if (items > INT32_MAX) return invalid("opm_update: too large");
    const dim3 grid((unsigned)items);
    stage_mark(s, 0);
    if (K % 128 == 0) {
        hipLaunchKernelGGL(opm_update_kernel<128>, grid, dim3(256), 0, s, a);
    } else if (K % 64 == 0) {
        hipLaunchKernelGGL(opm_update_kernel<64>, grid, dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL(opm_update_kernel<32>, grid, dim3(256), 0, s, a);
    }
    stage_mark(s, 1);
    return launch_status("opm_update");
}

extern "C" int clk_opm_outer(clk_stream stream, const clk_buffer* left, const clk_buffer* right,
                             const clk_buffer* wT, const clk_buffer* out) {
    const clk_buffer* bufs[] = {left, right, wT, out};
    const int types[] = {CLK_F16, CLK_F16, CLK_F16, CLK_F16};
    if (int st = check_types("opm_outer", bufs, types, 4)) return st;
    if (left->rank != 3 || right->rank != 3 || wT->rank != 2 || left->dims[0] != kOpmRows ||
        right->dims[0] != kOpmRows) {
        return invalid("opm_outer: left must be [16,B,C], right [16,D,E], wT [F,C*E]");
    }
    const int64_t B = left->dims[1], C = left->dims[2], D = right->dims[1], E = right->dims[2];
    const int64_t F = wT->dims[0];
    if (C % kOpmChunk || E != kOpmE || D % kOpmD || D / kOpmD > 65535 || wT->dims[1] != C * E ||
        !opm_width(F)) {
        return invalid("opm_outer: C a multiple of 16, E 32, D a multiple of 4, F 16, 32, 64 or 128");
    }
    if (elements(out) != B * D * F) return invalid("opm_outer: shapes do not match");
    if (B == 0 || D == 0 || C == 0) return ok();
    if (!aligned16(left->data) || !aligned16(wT->data) || !aligned16(out->data)) {
        return invalid("opm_outer: left, wT and out must be 16-byte aligned");
    }
    if (B > INT32_MAX || C > INT32_MAX) return invalid("opm_outer: too large");
    OpmOuterArgs a{static_cast<const half_t*>(left->data), static_cast<const half_t*>(right->data),
                   static_cast<const half_t*>(wT->data), static_cast<half_t*>(out->data), (int)B,
                   (int)C, (int)D};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    stage_mark(s, 0);
    const bool two = D % (2 * kOpmD) == 0;
    const dim3 grid((unsigned)((B + kOpmB - 1) / kOpmB), (unsigned)(D / (kOpmD * (two ? 2 : 1))));
#define CLK_OPM_OUTER(F_)                                                                              \
    if (two) hipLaunchKernelGGL((opm_outer_kernel<F_, 2>), grid, dim3(256), 0, s, a);                 \
    else hipLaunchKernelGGL((opm_outer_kernel<F_, 1>), grid, dim3(256), 0, s, a);
    switch (F) {
    case 16: CLK_OPM_OUTER(16) break;
    case 32: CLK_OPM_OUTER(32) break;
    case 64: CLK_OPM_OUTER(64) break;
    default: CLK_OPM_OUTER(128) break;
    }
#undef CLK_OPM_OUTER
    stage_mark(s, 1);
    return launch_status("opm_outer");
}
