// Flash-attention backward for gfx950 (CDNA4): dQ, dK, dV and a deterministic dBias.
//
// Semantics follow the reference's VoltaMmaBwd (cuda/volta_mma_attn_bwd.cu:84-451): P is rebuilt
// from the forward's log2-domain lse, p = exp2(s2 - lse2); a dead logit (masked key, or a query
// or key past the end) takes the masked logit -1e4, so P still carries dV for a masked key, while
// dS = p (dP - delta) is zero there; delta = rowsum(out * dout) in fp32 from the fp16 tensors
// (cuda/volta_attn_bwd.h:21-42); P and dS are fp16 before their GEMMs; dq = scale dS K and
// dk = scale dS^T Q accumulate in fp32 and round once; dbias = sum over the N rows of dS in fp32,
// unscaled, and all zeros without want_dbias (volta_mma_attn_bwd.cu:363).
//
// Where the reference adds dQ and dBias with fp32 atomics into global memory, this backward is
// three kernels with no atomics, so every result is bit-identical from run to run:
//   biast_kernel  log2e bias transposed to [H][keys][queries] (fp32, zero-padded), so a dK/dV
//                 lane reads its eight queries' bias at its key with two 16-byte loads and
//                 s2 = scale log2e S + log2e bias is one fma.
//   dq_kernel     one workgroup per (n, h, 128 queries), looping over key tiles as the forward
//                 does: dQ^T = K^T dS^T accumulates in registers; it also writes delta and lse2
//                 padded to whole 32-query tiles (0 and +inf past Sq).
//   dkdv_kernel   one workgroup per (h, 64 keys, chunk of batch rows): for each row n of its
//                 chunk it loops over query tiles, dV^T = dO^T P and dK^T = Q^T dS accumulate in
//                 registers, and each wave adds its 16 keys' dS into an fp32 [Sq][64 keys] dBias
//                 partial that stays in LDS for the whole chunk (one owner per element, fixed
//                 order). The chunk's partial goes to the workspace once.
//   dbias_kernel  dbias = the chunk partials summed in chunk order.
#include "clk_common.h"

#include <mutex>

namespace clk {

struct BwdArgs {
    const half_t* q;
    const half_t* k;
    const half_t* v;
    const half_t* bias;
    const uint8_t* kmask;
    const half_t* out;
    const half_t* dout;
    const float* lse;
    half_t* dq;
    half_t* dk;
    half_t* dv;
    float* dbias;
    // workspace [N, H, SqA / 32][64]: per 32-query tile, -lse2 / c1 of its queries (-inf past
    // Sq), then -rowsum(out * dout) of them (0 past Sq)
    float* qstat;
    // workspace [H, SkA + 1, SqB]: log2e bias[h][q][key] (fp32), -inf outside; row SkA of each
    // head holds the masked logit (log2e kMaskedLogit), the bias a dead key's lane reads
    float* biast;
    float* partial;  // workspace [chunks][H][kblocks][SqA][64]
    // workspace [H][SqA / 16][kblocks][2][64][8]: the dQ kernel's bias fragments. For each block
    // of 16 queries and 64-key tile, part 0 holds for lane l = r + 16 g the bias of query r, keys
    // 16 g .. +7, part 1 keys 16 g + 8 .. +15 (zero outside Sq and Sk), so that each of its bias
    // loads is one contiguous 1 KB sweep
    half_t* bfrag;
    // workspace [2][windows][N][H][Sk][D]: with more than one query window, each window's fp32
    // dK (unscaled) and dV sums over its queries, added up in window order by dkdv_sum_kernel
    float* dkv;
    int N, H, Sq, Sk, D;
    int SqA, SkA;    // Sq rounded up to 32, Sk rounded up to 64
    int SqB;         // queries per transposed-bias row: SqA, or 32 QT for the register kernel
    int kblocks;     // ceil(Sk / 64)
    int chunk;       // batch rows per dkdv workgroup
    int chunks;
    int wtiles;      // 32-query tiles per query window of the dK/dV kernel
    int windows;     // query windows: ceil(Sq / 32 / wtiles)
    float scale;
    float c1;    // scale log2e, or 1 where |scale log2e| is below 1e-30
    float c1s;   // c1 / log2e: scale, or the stand-in's 1 / log2e
    float rc1;   // 1 / c1
    int kscale;  // 0 where c1 stands in for a negligible scale: the dK/dV kernel's K is then zero
    int bias_vec;
    int dbias_vec;  // dbias rows are whole 16-byte vectors (Sk % 4 == 0, 16-byte aligned)
    // division by the dQ kernel's query tiles per (n, h), by N, kblocks, chunks and windows
    FastDiv fqt, fn, fkb, fch, fwin;
};

__device__ __forceinline__ half8 bzero8() {
    half8 z;
#pragma unroll
    for (int j = 0; j < 8; ++j) z[j] = (half_t)0.f;
    return z;
}

__device__ __forceinline__ half8 bld8(const half_t* p) { return *reinterpret_cast<const half8*>(p); }

struct BH16 {
    half8 lo, hi;
};

// ------------------------------------------------------------------------------------------
// dQ (and delta): the forward's orientation, S^T = K Q^T and dP^T = V dO^T with a lane on one
// query; dQ^T = K^T dS^T takes dS^T straight from registers as its B operand.
// ------------------------------------------------------------------------------------------
template <int DP>
struct DqTile {
    // at D <= 32 one 16-query block per wave (86 VGPRs: five waves per SIMD), else two
    static constexpr int kWaves = 4, kThreads = kWaves * kWave, kQB = DP == 32 ? 1 : 2;
    static constexpr int kBQ = kWaves * kQB * 16, kBK = 64;
    static constexpr int kKS = DP / 32, kDB = DP / 16;
    static constexpr int kLd = DP + 8;
    static constexpr int kChunks = kBK * DP / 8;
    static constexpr int kCPT = (kChunks + kThreads - 1) / kThreads;
};

// At D = 32 one query block per wave fits 86 VGPRs (five waves per SIMD), which measured 1-3%
// faster than two blocks at three waves per SIMD (142 VGPRs); four waves per workgroup (eight,
// sharing each key tile, measured 16% slower).
template <int DP>
__global__ __launch_bounds__(DqTile<DP>::kThreads, DP == 32 ? 4 : 1) void attn_bwd_dq_kernel(BwdArgs a) {
    using T = DqTile<DP>;
    // two key tiles in flight: one being read by the MFMAs, the next being written
    // (at DP = 32 four unpadded arrays instead, one per tensor and buffer: below)
    __shared__ __attribute__((aligned(16))) half_t Ks2[DP == 32 ? 1 : 2][T::kBK * T::kLd];
    __shared__ __attribute__((aligned(16))) half_t Vs2[DP == 32 ? 1 : 2][T::kBK * T::kLd];
    constexpr int kD32 = DP == 32 ? T::kBK * 32 : 8;
    __shared__ __attribute__((aligned(16))) half_t K32a[kD32], K32b[kD32], V32a[kD32], V32b[kD32];

    const int item = xcd_item(blockIdx.x, gridDim.x);
    // head-major order: an XCD's contiguous run of items covers few heads, so the bias rows
    // it reads stay in its L2
    const int rest = fdiv(item, a.fqt), qt = item - rest * (int)a.fqt.d;
    const int h = fdiv(rest, a.fn), n = rest - h * a.N;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int r16 = lane & 15, g = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int64_t nh = (int64_t)n * a.H + h;
    const int64_t qbase = nh * a.Sq * a.D, kbase = nh * a.Sk * a.D;
    const int q0w = qt * T::kBQ + wave * (T::kQB * 16);

    // Q^T and dO^T B operands, lse2 and delta of this lane's queries: buffer loads over the
    // (n, h) block of q, dout and out, whose out-of-range slots (past Sq, or d past D) read zeros
    half8 qop[T::kQB][T::kKS], dop[T::kQB][T::kKS];
    float lse2[T::kQB], dlt[T::kQB];
    const int qrange = __builtin_amdgcn_readfirstlane(a.Sq * a.D * 2);
    const auto rq = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.q + qbase), 0, qrange, 0x00020000);
    const auto rdo = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.dout + qbase), 0, qrange, 0x00020000);
    const auto ro = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.out + qbase), 0, qrange, 0x00020000);
    // (run after the first key tile's loads are issued, so that their latencies overlap)
    const auto load_queries = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int qb = 0; qb < T::kQB; ++qb) {
        const int gq = q0w + 16 * qb + r16;
        const bool in = gq < a.Sq;
        float part = 0.f;
#pragma unroll
        for (int ks = 0; ks < T::kKS; ++ks) {
            const int d0 = 32 * ks + 8 * g;
            const uint32_t voff = in && d0 < a.D ? (uint32_t)(gq * a.D + d0) * 2u : 0x80000000u;
            qop[qb][ks] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rq, voff, 0, 0));
            dop[qb][ks] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rdo, voff, 0, 0));
            const half8 o = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(ro, voff, 0, 0));
#pragma unroll
            for (int j = 0; j < 8; ++j) part += (float)o[j] * (float)dop[qb][ks][j];
        }
        dlt[qb] = wave_xor_sum4(part);
        // a query past Sq gets lse2 = +inf, so its p is 0 whatever its logits
        lse2[qb] = in ? a.lse[nh * a.Sq + gq] : INFINITY;
        if (gq < a.SqA && g == 0) {
            // the dK/dV kernel's accumulator inputs: -delta and -lse2 / c1 (past Sq the latter
            // is infinite with the sign that makes c1 times it -inf)
            float* st = a.qstat + (nh * a.SqA + (gq & ~31)) * 2 + (gq & 31);
            st[0] = (in ? -lse2[qb] : -INFINITY) * a.rc1;
            st[32] = in ? -dlt[qb] : 0.f;
        }
    }
    };

    float4v acc[T::kDB][T::kQB];
#pragma unroll
    for (int db = 0; db < T::kDB; ++db)
#pragma unroll
        for (int qb = 0; qb < T::kQB; ++qb) acc[db][qb] = float4v{0.f, 0.f, 0.f, 0.f};

    // K/V chunks of the next key tile, one tile ahead of their LDS store: fixed row and column
    // per lane, buffer loads whose range is the tile's rows below Sk (a row past Sk and a column
    // past D read zeros). The mask bytes run a tile further ahead: lane l of every wave loads the
    // byte of key k0 + l (zero past Sk) of the tile after the next, so a wave ballot of them (the
    // tile's keep bits, uniform across the workgroup) is known, with no wait, when that tile's K/V
    // loads are issued. A masked key's K row is staged as zeros.
    uint32_t kvoff[T::kCPT];
    int krow[T::kCPT], kdst[T::kCPT];
#pragma unroll
    for (int i = 0; i < T::kCPT; ++i) {
        const int c = tid + i * T::kThreads;  // kChunks = kCPT kThreads
        const int row = c / (DP / 8), col = (c - row * (DP / 8)) * 8;
        kvoff[i] = col < a.D ? (uint32_t)((row * a.D + col) * 2) : 0x80000000u;
        krow[i] = row;
        kdst[i] = perm_row(row, 16) * T::kLd + col;
    }
    const char* const kb_base = reinterpret_cast<const char*>(a.k + kbase);
    const char* const vb_base = reinterpret_cast<const char*>(a.v + kbase);
    const char* const mrow = reinterpret_cast<const char*>(a.kmask + (int64_t)n * a.Sk);
    half8 kreg[T::kCPT], vreg[T::kCPT];
    const auto fetch_mask = [&](int k0) -> uint32_t {
        const int rows = min(a.Sk - k0, T::kBK);
        const auto rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(mrow + k0), 0, rows, 0x00020000);
        return __builtin_amdgcn_raw_buffer_load_b8(rm, (uint32_t)lane, 0, 0);
    };
    const auto fetch = [&](int k0) {
        const int rows = min(a.Sk - k0, T::kBK);
        const int64_t kofs = (int64_t)k0 * a.D * 2;
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kb_base + kofs), 0, rows * a.D * 2, 0x00020000);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vb_base + kofs), 0, rows * a.D * 2, 0x00020000);
#pragma unroll
        for (int i = 0; i < T::kCPT; ++i) {
            kreg[i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rk, kvoff[i], 0, 0));
            vreg[i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rv, kvoff[i], 0, 0));
        }
    };
    // At DP = 32 the K and V tiles go from memory straight into LDS by direct-to-LDS loads
    // (buffer_load ... lds), one 1 KB load of each per wave, issued at the start of the previous
    // tile and complete at its closing barrier. Their rows are unpadded 64 bytes with the 16-byte
    // chunks of LDS row R at chunk position c ^ ((R / 4) % 4), so the row-form reads of 16
    // consecutive rows fall on 16 distinct bank groups: slot l of wave w's load is LDS row
    // R = 16 w + l / 4 (key x with perm_row(x, 16) = R), position l % 4. A masked key's K slots
    // take an offset past the buffer's range, so the load itself writes their zeros; the first
    // tile, loaded before its keep bits are known, is zeroed in LDS instead.
    uint32_t kvdma = 0u;
    int dkey = 0;
    if constexpr (DP == 32) {
        const int R = 16 * wave + (lane >> 2), pos = lane & 3;
        dkey = 16 * ((R >> 2) & 3) + 4 * (R >> 4) + (R & 3);
        const int col = 8 * (pos ^ ((R >> 2) & 3));
        kvdma = col < a.D ? (uint32_t)((dkey * a.D + col) * 2) : 0x80000000u;
    }
    const auto dma_kv = [&](int k0, int buf, uint64_t keep) {
        const int rows = min(a.Sk - k0, T::kBK);
        const int64_t kofs = (int64_t)k0 * a.D * 2;
        const int range = __builtin_amdgcn_readfirstlane(rows * a.D * 2);
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kb_base + kofs), 0, range, 0x00020000);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vb_base + kofs), 0, range, 0x00020000);
        const uint32_t koff = (keep >> dkey) & 1u ? kvdma : 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rk, (__attribute__((address_space(3))) void*)((buf ? K32b : K32a) + 512 * wv), 16, koff, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rv, (__attribute__((address_space(3))) void*)((buf ? V32b : V32a) + 512 * wv), 16, kvdma, 0, 0, 0);
    };
    const auto fetch_kv = [&](int k0, int buf, uint64_t keep) {
        if constexpr (DP == 32) {
            dma_kv(k0, buf, keep);
        } else {
            fetch(k0);
        }
    };
    // the register-staged tile into LDS buffer buf, masked K rows as zeros (DP != 32); at DP = 32
    // the zeroing of the first tile's masked K rows, once its loads have landed
    const auto stage = [&](int buf, uint64_t keep) {
        if constexpr (DP == 32) {
            if (keep != ~0ull) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                if (!((keep >> dkey) & 1u))
                    *reinterpret_cast<half8*>((buf ? K32b : K32a) + 512 * wv + 8 * lane) = bzero8();
            }
        } else {
#pragma unroll
            for (int i = 0; i < T::kCPT; ++i) {
                *reinterpret_cast<half8*>(&Ks2[buf][kdst[i]]) = (keep >> krow[i]) & 1u ? kreg[i] : bzero8();
                *reinterpret_cast<half8*>(&Vs2[buf][kdst[i]]) = vreg[i];
            }
        }
    };
    // LDS address of tile row r (after the row permutation), chunk 8 c: padded rows, or at DP = 32
    // the swizzled unpadded rows
    const auto kv_at = [&](const half_t* t, int R, int c) -> const half_t* {
        if constexpr (DP == 32) {
            return t + 32 * R + 8 * (c ^ ((R >> 2) & 3));
        } else {
            return t + R * T::kLd + 8 * c;
        }
    };

    const float scale = a.scale;

    // bias of this lane's 16 keys k0 + 16 g .. +15, one key tile ahead of their use, in two
    // register sets that alternate by tile; when the tile comes up, a masked key or a key past
    // Sk gets bias -inf, so its p, and with it its dS, is 0. The values come from the fragment
    // copy the transposed-bias kernel writes: per 16-query block and key tile two 1 KB parts in
    // lane order, read from a wave-uniform base (a block past SqA, whose queries are all past Sq,
    // reads the last real block instead).
    const int wq = __builtin_amdgcn_readfirstlane(q0w);
    const half_t* bfr[T::kQB];
#pragma unroll
    for (int qb = 0; qb < T::kQB; ++qb) {
        const int qblk = min((wq + 16 * qb) / 16, a.SqA / 16 - 1);
        bfr[qb] = a.bfrag + ((int64_t)h * (a.SqA / 16) + qblk) * a.kblocks * 1024;
    }
    const auto fetch_bias = [&](int k0, BH16 (&b)[T::kQB]) {
#pragma unroll
        for (int qb = 0; qb < T::kQB; ++qb) {
            b[qb].lo = bld8(bfr[qb] + (k0 / T::kBK) * 1024 + 8 * lane);
            b[qb].hi = bld8(bfr[qb] + (k0 / T::kBK) * 1024 + 512 + 8 * lane);
        }
    };
    const auto fix_bias = [&](int k0, BH16 (&b)[T::kQB], uint64_t keep64) {
        const int kvalid = a.Sk - (k0 + 16 * g);
        const uint32_t inside = kvalid >= 16 ? 0xffffu : kvalid <= 0 ? 0u : (1u << kvalid) - 1u;
        const uint32_t keep = (uint32_t)(keep64 >> (16 * g)) & inside;
        if (keep != 0xffffu) {
#pragma unroll
            for (int qb = 0; qb < T::kQB; ++qb)
                fill_bias16(b[qb].lo, b[qb].hi, keep, 0u, (half_t)(-INFINITY), (half_t)(-INFINITY));
        }
    };

    // dP^T starts from -delta (the MFMA accumulator input), so dS = p dP is one multiply
    float4v ndlt[T::kQB];

    // keep bits of this tile, and the mask byte of the next tile (loaded a tile ago)
    uint64_t keep_cur = 0u;
    uint32_t mbyte = 0u;
    const int k_last = a.Sk > 0 ? (a.Sk - 1) / T::kBK * T::kBK : 0;
    const auto tile = [&](int k0, int buf, BH16 (&bias16)[T::kQB], BH16 (&bias_next)[T::kQB]) {
        const half_t* Ks = DP == 32 ? (buf ? K32b : K32a) : Ks2[buf & (DP == 32 ? 0 : 1)];
        const half_t* Vs = DP == 32 ? (buf ? V32b : V32a) : Vs2[buf & (DP == 32 ? 0 : 1)];
        // the next tile's K, V and bias and the mask byte of the one after it, issued
        // unconditionally (past the last tile the last one again, unused): with no branch
        // around the loads the compiler knows how many are in flight, and no value they bring is
        // examined before the barrier that ends the tile, so they stay in flight until then
        const uint64_t keep_next = __ballot(mbyte != 0u);
        const int kn = min(k0 + T::kBK, k_last);
        fetch_kv(kn, buf ^ 1, keep_next);
        fetch_bias(kn, bias_next);
        mbyte = fetch_mask(min(k0 + 2 * T::kBK, k_last));
        // every key of the tile kept and inside Sk: the bias stands as loaded
        if (keep_cur != ~0ull) fix_bias(k0, bias16, keep_cur);

        // the tile in two halves of 32 keys: key blocks 2 kt and 2 kt + 1 hold keys 16 g + 8 kt + j,
        // which are the k-slots of dQ^T's contraction step kt, so each half's S^T and dP^T
        // registers are free again once its dS^T is packed
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            float4v s[2][T::kQB], dp[2][T::kQB];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                const int krw = 16 * (2 * kt + k2) + r16;  // key 16 (r/4) + 4 kb + r%4
#pragma unroll
                for (int qb = 0; qb < T::kQB; ++qb) {
                    s[k2][qb] = float4v{0.f, 0.f, 0.f, 0.f};
                    dp[k2][qb] = ndlt[qb];
                }
#pragma unroll
                for (int ks = 0; ks < T::kKS; ++ks) {
                    const half8 kop = bld8(kv_at(Ks, krw, 4 * ks + g));
                    const half8 vop = bld8(kv_at(Vs, krw, 4 * ks + g));
#pragma unroll
                    for (int qb = 0; qb < T::kQB; ++qb) {
                        s[k2][qb] = mfma16x16x32(kop, qop[qb][ks], s[k2][qb]);
                        dp[k2][qb] = mfma16x16x32(vop, dop[qb][ks], dp[k2][qb]);
                    }
                }
            }

            // dS^T = P^T (dP^T - delta), packed as the B operand of dQ^T; a dead logit has p = 0
            half8 dsb[T::kQB];
#pragma unroll
            for (int qb = 0; qb < T::kQB; ++qb) {
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int kk = 4 * (2 * kt + k2) + i;
                        const half_t b = kk < 8 ? bias16[qb].lo[kk] : bias16[qb].hi[kk - 8];
                        const float t = fmaf(s[k2][qb][i], scale, (float)b);
                        const float p = exp2_fast(fmaf(t, kLog2e, -lse2[qb]));
                        const float ds = p * dp[k2][qb][i];
                        dsb[qb][4 * k2 + i] = (half_t)pin_f32(ds);
                    }
                }
            }

#pragma unroll
            for (int db = 0; db < T::kDB; ++db) {
                // K^T read transposed from the row-major K tile: slots are keys 16 g + 8 kt + j
                half8 kto;
                if constexpr (DP == 32) {
                    const int j = r16 >> 2, c = r16 & 3;
                    const int Rl = perm_row(16 * g + 8 * kt + j, 16), Rh = perm_row(16 * g + 8 * kt + 4 + j, 16);
                    const half4 lo = lds_read_tr16(Ks + 32 * Rl + 8 * (c ^ ((Rl >> 2) & 3)) + 4 * db);
                    const half4 hi = lds_read_tr16(Ks + 32 * Rh + 8 * (c ^ ((Rh >> 2) & 3)) + 4 * db);
                    kto = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                } else {
                    kto = lds_operand_tr([&](int r) { return Ks + perm_row(r, 16) * T::kLd; },
                                         2 * g + kt, r16, 4 * db, DP / 4);
                }
#pragma unroll
                for (int qb = 0; qb < T::kQB; ++qb) acc[db][qb] = mfma16x16x32(kto, dsb[qb], acc[db][qb]);
            }
        }
        // (DP != 32) the next tile's registers into the other buffer, last read a tile ago,
        // before the barrier that ended that tile
        if constexpr (DP != 32) stage(buf ^ 1, keep_next);
        // every load of this tile has landed before the barrier after which the waves read the
        // next tile's K and V (the compiler also waits for all loads before a barrier; the order
        // does not rest on it), by a waitcnt the compiler sees, so it knows that nothing is in
        // flight past the barrier
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        __syncthreads();
        keep_cur = keep_next;
    };

    BH16 biasA[T::kQB], biasB[T::kQB];
    uint32_t mbyte0 = 0u;
    if (a.Sk > 0) {
        // the first tile's K and V before its keep bits are known (its masked K rows are zeroed
        // in LDS below), its bias, and the mask bytes of the first two tiles
        mbyte0 = fetch_mask(0);
        fetch_kv(0, 0, ~0ull);
        fetch_bias(0, biasA);
        mbyte = fetch_mask(min(T::kBK, k_last));
    }
    load_queries();
#pragma unroll
    for (int qb = 0; qb < T::kQB; ++qb) ndlt[qb] = float4v{-dlt[qb], -dlt[qb], -dlt[qb], -dlt[qb]};
    if (a.Sk > 0) {
        keep_cur = __ballot(mbyte0 != 0u);
        stage(0, keep_cur);
        // the prologue's loads (the first tile, Q, dO, O, lse) have all landed before the loop,
        // and the compiler knows it: the loop's waits then count only the loop's own loads
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        __syncthreads();
    }
    for (int k0 = 0; k0 < a.Sk; k0 += 2 * T::kBK) {
        tile(k0, 0, biasA, biasB);
        if (k0 + T::kBK < a.Sk) tile(k0 + T::kBK, 1, biasB, biasA);
    }

#pragma unroll
    for (int qb = 0; qb < T::kQB; ++qb) {
        const int gq = q0w + 16 * qb + r16;
        if (gq >= a.Sq) continue;
#pragma unroll
        for (int c = 0; c < DP / 32; ++c) {
            const int d0 = (DP / 4) * g + 8 * c;
            if (d0 >= a.D) continue;
            half8 o;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = (half_t)(acc[2 * c + j / 4][qb][j & 3] * scale);
            *reinterpret_cast<half8*>(a.dq + qbase + (int64_t)gq * a.D + d0) = o;
        }
    }
}

// ------------------------------------------------------------------------------------------
// dK, dV and the dBias partials: S = Q K^T and dP = dO V^T with a lane on one key, so P and dS
// feed dV^T = dO^T P and dK^T = Q^T dS as B operands straight from registers.
//
// A workgroup owns 64 keys (four key groups of 16, one wave each) and QG row groups of its chunk
// of batch rows: row group rg takes rows n_begin + rg, + QG, ..., and for each row walks all of
// its query tiles of 32, staged by its four waves into its own pair of LDS buffers (one read, one
// being written, one barrier per step). A row's dK and dV therefore accumulate in one wave's
// registers with no cross-wave sum. The row groups walk the tiles of a row from staggered
// starting tiles, so at every step they add dS into disjoint columns of the fp32 [64 keys][Sq]
// dBias partial that stays in LDS for the whole chunk: each element is updated by one wave per
// step, in an order fixed by the schedule.
//
// The per-query terms enter the MFMAs as accumulator inputs: S starts from -lse2 / (scale log2e)
// and dP from -delta (a lane loads one of its 16-lane row's sixteen terms with the tile's chunks
// and the row shares them by DPP broadcasts), so that s2 = scale log2e S + bias log2e
// is one fma and dS = p dP one multiply. A dead key (masked, or past Sk) has zero K and V rows and
// the masked logit in place of its bias, so p still carries dV; its dS is set to 0. Both happen
// on a path that only waves holding a dead key take.
// ------------------------------------------------------------------------------------------
// LDS layout of the dK/dV kernel's Q and dO tiles (32 rows of DP halfs), in 4-byte words: panels
// of 32 columns, 512 words each; in a panel LDS row R takes 16 words, with its 16-byte chunk k at
// chunk k ^ 2 (m / 2) and the 8-byte half h of a chunk at half h ^ (m % 2), m = (R / 4) % 4.
// gfx950's LDS serves 8-byte reads 32 lanes at a time from 64 banks; with this layout the
// kernel's two 8-byte read shapes, 16 rows of one chunk (the row-form A operands, two reads)
// and 8 rows x 4 chunks (the transpose reads), fall on distinct banks. `col` is a multiple of 4.
__device__ __forceinline__ int dkdv_word(int R, int col) {
    const int p = col >> 5, k = (col >> 3) & 3, h = (col >> 2) & 1, m = (R >> 2) & 3;
    return 512 * p + 16 * R + 4 * (k ^ (2 * (m >> 1))) + 2 * (h ^ (m & 1));
}

// The transposed MFMA operand of d block db from a tile in that layout: A row r of the block is
// d = 32 (db / 2) + 8 (r / 4) + 4 (db % 2) + r % 4, its k-slot j tile row 8 g + j (at LDS row
// perm_row(8 g + j, 8)); two transpose reads of 4 rows each.
__device__ __forceinline__ half8 dkdv_operand_tr(const half_t* tile, int g, int lane16, int db) {
    const int j = lane16 >> 2, c = lane16 & 3;
    const int col = 32 * (db >> 1) + 4 * (db & 1) + 8 * c;
    const half4 lo = lds_read_tr16(tile + 2 * dkdv_word(perm_row(8 * g + j, 8), col));
    const half4 hi = lds_read_tr16(tile + 2 * dkdv_word(perm_row(8 * g + 4 + j, 8), col));
    return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Lanes B .. B + 3 of this lane's 16-lane row (DPP row broadcasts).
template <int B>
__device__ __forceinline__ float4v row_quad(float v) {
    const int x = __builtin_bit_cast(int, v);
    return float4v{__builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x150 + B, 0xf, 0xf, true)),
                   __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x151 + B, 0xf, 0xf, true)),
                   __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x152 + B, 0xf, 0xf, true)),
                   __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x153 + B, 0xf, 0xf, true))};
}

template <int DP, int QG>
struct DkdvTile {
    static constexpr int kWaves = 4 * QG, kThreads = kWaves * kWave;
    static constexpr int kBK = 64;                    // keys per workgroup, 16 per key group
    static constexpr int kBQ = 32;                    // queries per tile (one contraction step)
    static constexpr int kKS = DP / 32, kDB = DP / 16;
    static constexpr int kTile = kBQ * DP;            // halfs of a Q or dO tile
    static constexpr int kChunks = 2 * kBQ * DP / 8;  // Q and dO chunks of one tile
    static constexpr int kCPT = (kChunks + 255) / 256;
    // halfs per row group and buffer: the Q tile, 128 bytes of gap, then the dO tile (the gap
    // keeps the compiler from pairing a Q read with the dO read at the same offset into one
    // two-address read, whose halves would then need register moves)
    static constexpr int kOs = kTile + 64;
    static constexpr int kStage = kOs + kTile;
    static constexpr int kStageBytes = kStage * 2 * 2 * QG;  // two buffers per row group
};

template <int DP, int QG, bool DBIAS>
__global__ __launch_bounds__(256 * QG) void attn_bwd_dkdv_kernel(BwdArgs a) {
    using T = DkdvTile<DP, QG>;
    extern __shared__ __attribute__((aligned(16))) char lds_raw[];

    const int item = xcd_item(blockIdx.x, gridDim.x);
    // head-major order, as in the forward: an XCD's run of items reads few heads' bias columns;
    // the key blocks of one query window and chunk are neighbours, so they share Q and dO in L2
    const int rest = fdiv(item, a.fkb), kblk = item - rest * a.kblocks;
    const int rest2 = fdiv(rest, a.fwin), win = rest - rest2 * a.windows;
    const int h = fdiv(rest2, a.fch), c = rest2 - h * a.chunks;
    const int n_begin = c * a.chunk;
    const int n_end = min(a.N, n_begin + a.chunk);
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    // the wave index as a scalar: a row group's rows, tiles and step decisions are then uniform
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int kg = wave & 3, rg = wave >> 2, gtid = tid & 255;
    const int r16 = lane & 15, g = lane >> 4;
    const int klocal = kg * 16 + r16;
    const int key = kblk * T::kBK + klocal;
    const bool kin = key < a.Sk;
    // this workgroup's query window: tiles wt0 .. wt0 + qtiles - 1 (at least QG of them, the
    // host plans QG so); tile indices below are within the window
    const int wt0 = win * a.wtiles;
    const int qtiles = min(a.wtiles, (a.Sq + T::kBQ - 1) / T::kBQ - wt0);
    const int qsteps = (qtiles + 1) & ~1;            // steps per row: even, an odd count padded
    const int stagger = qtiles / QG;                 // tile offset between row groups
    const int rows = (n_end - n_begin + QG - 1) / QG;  // row passes of the busiest row group

    half_t* const stage0 = reinterpret_cast<half_t*>(lds_raw) + rg * T::kStage;
    constexpr int kBufStride = QG * T::kStage;  // halfs from buffer 0 to buffer 1 of a group
    // dBias partial of the window [32 qtiles / 4][kBK keys][4 queries]: a 16-lane group's four
    // queries of 16 keys are one contiguous 256 bytes
    float* DBt = reinterpret_cast<float*>(lds_raw + T::kStageBytes);

    if constexpr (DBIAS) {
        for (int i = tid; i < T::kBK * T::kBQ * qtiles; i += T::kThreads) DBt[i] = 0.f;
    }

    const float scale = a.scale;
    const float c1 = a.c1;  // scale log2e, or the stand-in for a negligible scale (K is zero then)

    // Step `it` of a row pass is query tile tile_of(it) of the group's row for that pass; a step
    // past the row's tiles, or a pass past n_end, is idle. Every load below is issued
    // unconditionally, from a scalar base and a lane offset fixed for the kernel, and judged
    // only where it is used, so the loop body is straight-line and each wait covers exactly the
    // loads it needs.
    const auto tile_of = [&](int it) {
        const int x = (it < qtiles ? it : 0) + rg * stagger;
        return x >= qtiles ? x - qtiles : x;
    };
    // This lane's Q / dO chunks of a tile: a fixed row and column of a fixed source, Q or dO,
    // that is the same across a wave. The chunks are read with buffer loads whose range is the
    // tile's rows below Sq, so a row past Sq, a column past D and an idle step all read zeros.
    uint32_t cvoff[T::kCPT];
    int cdst0[T::kCPT], cdst1[T::kCPT];  // LDS halfs of the chunk's two 8-byte halves
    bool cdo[T::kCPT];
#pragma unroll
    for (int i = 0; i < T::kCPT; ++i) {
        const int cc = gtid + i * 256;  // every (Q, dO) x row x column chunk: kChunks = 256 kCPT
        const int which = cc / (T::kBQ * DP / 8), w = cc - which * (T::kBQ * DP / 8);
        const int row = w / (DP / 8), col = (w - row * (DP / 8)) * 8;
        cvoff[i] = col < a.D ? (uint32_t)((row * a.D + col) * 2) : 0x80000000u;
        cdst0[i] = which * T::kOs + 2 * dkdv_word(perm_row(row, 8), col);
        cdst1[i] = which * T::kOs + 2 * dkdv_word(perm_row(row, 8), col + 4);
        cdo[i] = (64 * (wave & 3) + 256 * i) / (T::kBQ * DP / 8) != 0;  // 4 DP is a multiple of 64
    }
    // one of the tile's query terms, [-lse2 / c1 of its 32 queries][-delta of them]: lane i of
    // 16-lane row g holds -lse2 / c1 of query 8 g + i for i < 8, -delta of query 8 g + i - 8 above
    const uint32_t st_off = 4u * (uint32_t)(r16 < 8 ? 8 * g + r16 : T::kBQ + 8 * g + r16 - 8);
    // this lane's eight queries' log2e bias at its key
    const char* const bt_base =
        reinterpret_cast<const char*>(a.biast + ((int64_t)h * (a.SkA + 1) + kblk * T::kBK) * a.SqB);
    const uint32_t bt_off = (uint32_t)(klocal * a.SqB + 8 * g) * 4u;

    // A step's Q / dO chunks: two register sets, one per step parity, fetched two steps ahead of
    // their stage. The bias and the query term: two register sets likewise, two steps ahead of
    // their use. (Padded past Sq: -lse2 / c1 infinite, -delta 0, bias 0.)
    struct Chunks {
        half8 s[T::kCPT];
    };
    Chunks ch0, ch1;
    float8v bt0, bt1;
    float sq0, sq1;
    // The chunk and bias prefetches walk the steps with cursors of their own, ahead of the
    // step being computed; a cursor past the last pass reads zeros (chunks) or a valid tile
    // (bias), unused.
    int cs_pass = 0, cs_it = 0, cs_tile = tile_of(0);
    bool cs_rowv = false;
    const char *cs_q = nullptr, *cs_o = nullptr;
    const auto cs_row = [&]() {
        const int n = n_begin + rg + QG * cs_pass;
        cs_rowv = n < n_end;
        const int64_t nh = (int64_t)(cs_rowv ? n : n_begin) * a.H + h;
        cs_q = reinterpret_cast<const char*>(a.q + nh * a.Sq * a.D);
        cs_o = reinterpret_cast<const char*>(a.dout + nh * a.Sq * a.D);
    };
    const auto fetch_s = [&](Chunks& d) {
        const int q0 = (wt0 + cs_tile) * T::kBQ;
        const bool v = cs_rowv && cs_it < qtiles;
        const int bytes = v ? min(T::kBQ, a.Sq - q0) * a.D * 2 : 0;
#pragma unroll
        for (int i = 0; i < T::kCPT; ++i) {
            const char* src = (cdo[i] ? cs_o : cs_q) + q0 * a.D * 2;
            const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(src), 0, bytes, 0x00020000);
            d.s[i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rs, cvoff[i], 0, 0));
        }
        if (++cs_it == qsteps) {
            cs_it = 0;
            ++cs_pass;
            cs_row();
        }
        cs_tile = tile_of(cs_it);
    };
    int bc_pass = 0, bc_it = 0;
    const char* bc_st = nullptr;
    const auto bc_row = [&]() {
        const int n = n_begin + rg + QG * bc_pass;
        const int64_t nh = (int64_t)(n < n_end ? n : n_begin) * a.H + h;
        bc_st = reinterpret_cast<const char*>(a.qstat + nh * a.SqA * 2);
    };
    const auto fetch_c = [&](float8v& d, float& sq) {
        const int q0 = (wt0 + tile_of(bc_it)) * T::kBQ;
        d = *reinterpret_cast<const float8v*>(bt_base + q0 * 4 + bt_off);
        sq = *reinterpret_cast<const float*>(bc_st + q0 * 8 + st_off);
        if (++bc_it == qsteps) {
            bc_it = 0;
            ++bc_pass;
            bc_row();
        }
    };
    const auto stage_tile = [&](const Chunks& d, int buf) {
        half_t* Qs = stage0 + buf * kBufStride;
#pragma unroll
        for (int i = 0; i < T::kCPT; ++i) {
            *reinterpret_cast<half4*>(Qs + cdst0[i]) = half4{d.s[i][0], d.s[i][1], d.s[i][2], d.s[i][3]};
            *reinterpret_cast<half4*>(Qs + cdst1[i]) = half4{d.s[i][4], d.s[i][5], d.s[i][6], d.s[i][7]};
        }
    };

    // K and V of this group's next row as the B operands (lane column = key, slots
    // d = 32 ks + 8 g + j) and the key's raw mask byte; both operands become zero for a dead key
    // when the row comes up
    half8 kopn[T::kKS], vopn[T::kKS];
    uint32_t mbn = 0u;
    const auto fetch_kv = [&](int pass) {
        const int n = n_begin + rg + QG * pass;
        const int64_t nh = (int64_t)(n < n_end ? n : n_begin) * a.H + h;
        const int kc = kin ? key : 0;
        mbn = (uint32_t)a.kmask[(int64_t)(n < n_end ? n : n_begin) * a.Sk + kc];
#pragma unroll
        for (int ks = 0; ks < T::kKS; ++ks) {
            const int d0 = 32 * ks + 8 * g;
            const int64_t off = nh * a.Sk * a.D + (int64_t)kc * a.D + (d0 < a.D ? d0 : 0);
            kopn[ks] = bld8(a.k + off);
            vopn[ks] = bld8(a.v + off);
        }
    };

    half8 kop[T::kKS], vop[T::kKS];
    bool alive = false, all_alive = true, nv = false;
    float4v accv[T::kDB], acck[T::kDB];

    cs_row();
    bc_row();
    if (rows > 0) {
        fetch_kv(0);
        fetch_s(ch0);
        fetch_s(ch1);
        fetch_c(bt0, sq0);
        fetch_c(bt1, sq1);
        stage_tile(ch0, 0);
        fetch_s(ch0);
    }
    __syncthreads();

    // step (pass, it) reads LDS buffer it & 1 and the bias set of its parity, which it refills
    // with the step two on once consumed; after its S and dP products it stages the next step
    // from the chunk set of that parity and refills the set with the step three on (steps past
    // the end load the last step again, unused)
    const auto step = [&](int it, Chunks& next, float8v& bt, float& sq) {
        const int buf = it & 1, q0 = tile_of(it) * T::kBQ;  // within the window
        const bool valid = nv && it < qtiles;
        const half_t* Qs = stage0 + buf * kBufStride;
        const half_t* Os = Qs + T::kOs;

        // The S and dP products, the exp and dS run on every step (an idle step reads zeros
        // from its staged tile and finite query terms, and its results are dropped), so the
        // step's prefetch and staging sit in straight-line code between them; only the
        // accumulations are skipped on an idle step.
        // This lane's dBias partial elements are read first, ahead of the S and dP products (the
        // row groups' tiles are disjoint at every step, also on idle steps, and this lane is the
        // only writer of these eight elements within its group; LDS float atomics measured
        // several times slower).
        float* dbrow = DBt + (q0 / 4 + 2 * g) * (4 * T::kBK) + 4 * klocal;
        float4 dblo, dbhi;
        if constexpr (DBIAS) {
            dblo = *reinterpret_cast<float4*>(dbrow);
            dbhi = *reinterpret_cast<float4*>(dbrow + 4 * T::kBK);
        }
        // S (from -lse2 / c1) and dP (from -delta): A row r of query block qb is query
        // 8 (r/4) + 4 qb + r%4 of the tile, so the lane holds queries 8 g + 4 qb + i
        float x[8];
        float4v dp[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const int qrow = 16 * qb + r16;
            float4v s = qb == 0 ? row_quad<0>(sq) : row_quad<4>(sq);
            dp[qb] = qb == 0 ? row_quad<8>(sq) : row_quad<12>(sq);
#pragma unroll
            for (int ks = 0; ks < T::kKS; ++ks) {
                const int w0 = 2 * dkdv_word(qrow, 32 * ks + 8 * g);
                const int w1 = 2 * dkdv_word(qrow, 32 * ks + 8 * g + 4);
                const half4 q0v = *reinterpret_cast<const half4*>(Qs + w0);
                const half4 q1v = *reinterpret_cast<const half4*>(Qs + w1);
                const half4 o0v = *reinterpret_cast<const half4*>(Os + w0);
                const half4 o1v = *reinterpret_cast<const half4*>(Os + w1);
                const half8 qa = half8{q0v[0], q0v[1], q0v[2], q0v[3], q1v[0], q1v[1], q1v[2], q1v[3]};
                const half8 oa = half8{o0v[0], o0v[1], o0v[2], o0v[3], o1v[0], o1v[1], o1v[2], o1v[3]};
                s = mfma16x16x32(qa, kop[ks], s);
                dp[qb] = mfma16x16x32(oa, vop[ks], dp[qb]);
            }
            // s2 = scale log2e S + log2e bias; a dead key (K zero) takes the masked logit
#pragma unroll
            for (int i = 0; i < 4; ++i) x[4 * qb + i] = fmaf(s[i], c1, bt[4 * qb + i]);
            if (!all_alive) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[4 * qb + i] = alive ? x[4 * qb + i] : fmaf(s[i], c1, kMaskedLogit2);
                }
            }
        }
        fetch_c(bt, sq);  // the bias and query term two steps on, into the registers just consumed
        // the other buffer was last read a step ago, before the barrier that ended that step
        stage_tile(next, buf ^ 1);
        fetch_s(next);  // the chunks three steps on

        half8 pb, dsb;
        float dsf[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float p = exp2_fast(x[j]);
            dsf[j] = pin_f32(p * dp[j >> 2][j & 3]);
            pb[j] = (half_t)p;
        }
        if (!all_alive) {
            // a dead key's dS is 0 (its p, from the masked logit, still carries dV)
#pragma unroll
            for (int j = 0; j < 8; ++j) dsf[j] = alive ? dsf[j] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) dsb[j] = (half_t)dsf[j];
        if (valid) {
            if constexpr (DBIAS) {
                dblo.x += dsf[0]; dblo.y += dsf[1]; dblo.z += dsf[2]; dblo.w += dsf[3];
                dbhi.x += dsf[4]; dbhi.y += dsf[5]; dbhi.z += dsf[6]; dbhi.w += dsf[7];
                *reinterpret_cast<float4*>(dbrow) = dblo;
                *reinterpret_cast<float4*>(dbrow + 4 * T::kBK) = dbhi;
            }

            // dV^T += dO^T P, dK^T += Q^T dS: A row r of d block db is
            // d = 32 (db/2) + 8 (r/4) + 4 (db%2) + r%4, its k-slots queries 8 g + j, read transposed
#pragma unroll
            for (int db = 0; db < T::kDB; ++db) {
                const half8 ot = dkdv_operand_tr(Os, g, r16, db);
                const half8 qt = dkdv_operand_tr(Qs, g, r16, db);
                accv[db] = mfma16x16x32(ot, pb, accv[db]);
                acck[db] = mfma16x16x32(qt, dsb, acck[db]);
            }
        }
        __syncthreads();
    };

    for (int pass = 0; pass < rows; ++pass) {
        const int n = n_begin + rg + QG * pass;
        nv = n < n_end;
        alive = nv && kin && mbn != 0u;
#pragma unroll
        for (int ks = 0; ks < T::kKS; ++ks) {
            kop[ks] = alive && a.kscale && 32 * ks + 8 * g < a.D ? kopn[ks] : bzero8();
            vop[ks] = alive && 32 * ks + 8 * g < a.D ? vopn[ks] : bzero8();
        }
        all_alive = __all(alive);
#pragma unroll
        for (int db = 0; db < T::kDB; ++db) {
            accv[db] = float4v{0.f, 0.f, 0.f, 0.f};
            acck[db] = float4v{0.f, 0.f, 0.f, 0.f};
        }
        fetch_kv(pass + 1 < rows ? pass + 1 : pass);

        for (int it = 0; it < qsteps; it += 2) {
            step(it, ch1, bt0, sq0);
            step(it + 1, ch0, bt1, sq1);
        }

        if (nv && kin) {
            // the row is done: lane holds d = 32 cc + 8 g .. + 8 of its key for each panel cc
            const int64_t off = ((int64_t)n * a.H + h) * a.Sk * a.D + (int64_t)key * a.D;
            if (a.windows == 1) {
#pragma unroll
                for (int cc = 0; cc < DP / 32; ++cc) {
                    const int d0 = 32 * cc + 8 * g;
                    if (d0 >= a.D) continue;
                    half8 ok, ov;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        ok[j] = (half_t)(acck[2 * cc + j / 4][j & 3] * scale);
                        ov[j] = (half_t)accv[2 * cc + j / 4][j & 3];
                    }
                    *reinterpret_cast<half8*>(a.dk + off + d0) = ok;
                    *reinterpret_cast<half8*>(a.dv + off + d0) = ov;
                }
            } else {
                // this window's sums, fp32, for dkdv_sum_kernel
                const int64_t plane = (int64_t)a.N * a.H * a.Sk * a.D;
                float* pk = a.dkv + win * plane + off;
                float* pv = a.dkv + (a.windows + win) * plane + off;
#pragma unroll
                for (int cc = 0; cc < DP / 32; ++cc) {
                    const int d0 = 32 * cc + 8 * g;
                    if (d0 >= a.D) continue;
#pragma unroll
                    for (int j = 0; j < 8; j += 4) {
                        *reinterpret_cast<float4*>(pk + d0 + j) =
                            make_float4(acck[2 * cc + j / 4][0], acck[2 * cc + j / 4][1],
                                        acck[2 * cc + j / 4][2], acck[2 * cc + j / 4][3]);
                        *reinterpret_cast<float4*>(pv + d0 + j) =
                            make_float4(accv[2 * cc + j / 4][0], accv[2 * cc + j / 4][1],
                                        accv[2 * cc + j / 4][2], accv[2 * cc + j / 4][3]);
                    }
                }
            }
        }
    }

    if constexpr (DBIAS) {
        // the window's rows of the chunk's [SqA][64] partial
        float* dst = a.partial + (((int64_t)c * a.H + h) * a.kblocks + kblk) * a.SqA * T::kBK +
                     (int64_t)wt0 * T::kBQ * T::kBK;
        for (int i = tid; i < qtiles * T::kBQ * T::kBK; i += T::kThreads) {
            const int q = i / T::kBK, kk = i % T::kBK;
            dst[i] = DBt[(q >> 2) * (4 * T::kBK) + 4 * kk + (q & 3)];
        }
    }
}

// ------------------------------------------------------------------------------------------
// dK, dV and the dBias partials where D == 32 and Sq <= 32 QT (QT = 4 launches it; the same
// layout in query parts, attn_bwd_dkdv_reg3_kernel, serves QT 8 and 12): the same
// products and lane layout as attn_bwd_dkdv_kernel, arranged so that the dBias partial never
// leaves registers. A workgroup of eight waves owns 64 keys of one head and a chunk of batch
// rows: wave w takes key group w % 4 (16 keys) and query half w / 4 (QT / 2 tiles of 32), so the
// dBias partial of its keys over its queries is QT / 2 x 8 registers per lane for the whole
// chunk. The two halves' dK and dV sums of a row meet in LDS once per row (one fixed order). The
// workgroup's transposed log2e bias (64 keys plus the masked-logit row, the same for every row)
// is read into LDS once, so the per-tile bias reads are LDS reads.
//
// The query loop is unrolled (every register index is static) and branch-free. The transposed
// bias is -inf for every query past Sq up to 32 QT, so a padded or absent query has p = 0 and
// dS = 0 whatever its (zero) Q, dO and query terms. A dead key (masked, or past Sk) needs no
// selects either: its lane reads the masked-logit bias row instead of its own (so with K zero its
// s2 is the masked logit's), and reads its -delta from a zeroed LDS area (so with V zero its dP,
// and with it dS, is exactly 0 while p still carries dV).
//
// Per step (two tiles per query half), in order: stage the next step (loaded a step ago) into the
// other LDS buffer, issue the loads of the step after it, compute the step, barrier. The query
// terms -lse2 / c1 and -delta of the step's tiles are staged beside them and read back as
// float4 broadcasts (the MFMA accumulator inputs of S and dP).
// ------------------------------------------------------------------------------------------
// The register kernel's Q and dO tiles (32 rows of 32 halfs), in 4-byte words: LDS row R takes 16
// words, its 16-byte chunk k at chunk k ^ ((R / 4) % 4), in order within the chunk. A row-form
// operand (16 rows of one chunk per 16 lanes) is then one conflict-free 16-byte read.
__device__ __forceinline__ int reg_word(int R, int col) {
    return 16 * R + 4 * ((col >> 3) ^ ((R >> 2) & 3)) + 2 * ((col >> 2) & 1);
}

// dkdv_operand_tr for the register kernel's layout (D = 32, d block db of 2)
__device__ __forceinline__ half8 reg_operand_tr(const half_t* tile, int g, int lane16, int db) {
    const int j = lane16 >> 2, c = lane16 & 3;
    const int col = 4 * db + 8 * c;
    const half4 lo = lds_read_tr16(tile + 2 * reg_word(perm_row(8 * g + j, 8), col));
    const half4 hi = lds_read_tr16(tile + 2 * reg_word(perm_row(8 * g + 4 + j, 8), col));
    return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

template <int QT>
struct RegTile {
    static constexpr int DP = 32;
    static constexpr int HT = QT / 2;                // tiles per query half
    static constexpr int kSteps = HT / 2;            // steps per row, two tiles per half each
    static constexpr int kTile = 32 * DP;            // halfs of a 32-query Q (or dO) tile
    static constexpr int kOs = kTile + 64;           // the dO tile, after a 128-byte gap
    static constexpr int kSub = kOs + kTile;         // halfs of one tile's Q and dO
    static constexpr int kBuf = 4 * kSub;            // halfs of a step: [half][tile]
    static constexpr int SqB = 32 * QT;              // transposed-bias row length
    static constexpr int kBRow = SqB + 4;            // its LDS row stride (floats)
    static constexpr int kSlots = kSteps == 1 ? 2 : 1;  // dK/dV meeting slots, by row parity
    static constexpr int kLdsBytes = 65 * kBRow * 4 + 2 * kBuf * 2 + 1024 * 4 + kSlots * 4 * 4 * 64 * 16;
};

template <int QT, bool DBIAS>
__global__ __launch_bounds__(512, 2) void attn_bwd_dkdv_reg_kernel(BwdArgs a) {
    using T = RegTile<QT>;
    static_assert(QT % 4 == 0 && QT <= 12, "whole steps of two tiles per half");
    constexpr int DP = T::DP, HT = T::HT, kSteps = T::kSteps, kSub = T::kSub, kOs = T::kOs;
    constexpr int kBuf = T::kBuf, SqB = T::SqB, kBRow = T::kBRow;
    __shared__ __attribute__((aligned(16))) float bias_l[65 * kBRow];  // rows: 64 keys, masked
    __shared__ __attribute__((aligned(16))) half_t lds[2 * kBuf];
    // query terms [buf][half][tile][-lse2 / c1 x 32, -delta x 32], then 512 zeros
    __shared__ __attribute__((aligned(16))) float qterms[1024];
    // the query half 1 waves' dK / dV sums of a row: [slot][key group][float4 j][lane]
    __shared__ __attribute__((aligned(16))) float4 red[T::kSlots * 4 * 4 * 64];

    const int item = xcd_item(blockIdx.x, gridDim.x);
    // head-major order: an XCD's run of items reads few heads' bias columns
    const int rest = fdiv(item, a.fkb), kblk = item - rest * a.kblocks;
    const int h = fdiv(rest, a.fch), c = rest - h * a.chunks;
    const int n_begin = c * a.chunk;
    const int rows = min(a.N, n_begin + a.chunk) - n_begin;
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int kg = wave & 3, qh = wave >> 2;
    const int r16 = lane & 15, g = lane >> 4;
    const int klocal = kg * 16 + r16;
    const int key = kblk * 64 + klocal;
    const bool kin = key < a.Sk;
    const float c1 = a.c1;

    // the workgroup's transposed bias: rows kblk 64 .. + 63 and the masked-logit row SkA
    {
        const float* src = a.biast + (int64_t)h * (a.SkA + 1) * SqB;
        for (int idx = tid; idx < 65 * (SqB / 4); idx += 512) {
            const int r = idx / (SqB / 4), c4 = idx - r * (SqB / 4);
            const int srow = r < 64 ? kblk * 64 + r : a.SkA;
            *reinterpret_cast<float4*>(bias_l + r * kBRow + 4 * c4) =
                *reinterpret_cast<const float4*>(src + (int64_t)srow * SqB + 4 * c4);
        }
    }
    if (tid < 128) reinterpret_cast<float4*>(qterms + 512)[tid] = make_float4(0.f, 0.f, 0.f, 0.f);

    // this wave's staging share of a step: tile (half sqh, tile si) of tensor (Q, dO), scalars,
    // rows crow and crow + 16 at a fixed column
    const int ti = wave >> 1, tensor = wave & 1, sqh = ti >> 1, si = ti & 1;
    const int crow = lane >> 2, ccol = (lane & 3) * 8;
    const uint32_t cvoff = (uint32_t)((crow * DP + ccol) * 2);
    const int cdst0 = (2 * sqh + si) * kSub + tensor * kOs + 2 * reg_word(perm_row(crow, 8), ccol);
    const int cdst1 = (2 * sqh + si) * kSub + tensor * kOs + 2 * reg_word(perm_row(crow + 16, 8), ccol);
    const half_t* const csrc = tensor ? a.dout : a.q;
    // wave 0 also stages the step's query terms: lane l, tile l / 16 of [half][tile], 4 floats
    const int qt_t = lane >> 4;
    const uint32_t qt_f = (uint32_t)(4 * (lane & 15));

    // row `pass` of the chunk, clamped to a real row past the end (its data is staged, never read)
    const auto row_n = [&](int pass) -> int { return n_begin + (pass < rows ? pass : 0); };
    const auto row_nh = [&](int pass) -> int64_t { return (int64_t)row_n(pass) * a.H + h; };
    half8 chk[2];
    float4 qst;
    const auto fetch_s = [&](int pass, int step) {
        const int64_t nh = row_nh(pass);
        const int q0 = 32 * (sqh * HT + 2 * step + si);
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<half_t*>(csrc + (nh * a.Sq + q0) * DP), 0, max(a.Sq - q0, 0) * DP * 2, 0x00020000);
        chk[0] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rs, cvoff, 0, 0));
        chk[1] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rs, cvoff + 16u * DP * 2u, 0, 0));
        if (wave == 0) {
            const int tg = (qt_t >> 1) * HT + 2 * step + (qt_t & 1);
            const auto rq = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(a.qstat + nh * a.SqA * 2), 0, a.SqA * 2 * 4, 0x00020000);
            qst = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                rq, ((uint32_t)(64 * tg) + qt_f) * 4u, 0, 0));
        }
    };
    const auto stage = [&](int buf) {
        half_t* dst = lds + buf * kBuf;
        *reinterpret_cast<half8*>(dst + cdst0) = chk[0];
        *reinterpret_cast<half8*>(dst + cdst1) = chk[1];
        if (wave == 0) *reinterpret_cast<float4*>(qterms + buf * 256 + 4 * lane) = qst;
    };

    // K and V of the next row as B operands (lane column = key, slots d = 8 g + j), its mask byte
    // the lane's K/V chunk and mask byte of a row: buffer loads from the row's (scalar) base at
    // offsets fixed for the kernel
    half8 kopn, vopn;
    uint32_t mbn = 0u;
    const uint32_t kvoff = (uint32_t)((kin ? key : 0) * DP + 8 * g) * 2u, moff = (uint32_t)(kin ? key : 0);
    const auto fetch_kv = [&](int pass) {
        const int64_t nh = row_nh(pass);
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.k + nh * a.Sk * DP), 0, a.Sk * DP * 2, 0x00020000);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.v + nh * a.Sk * DP), 0, a.Sk * DP * 2, 0x00020000);
        const auto rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.kmask + (int64_t)row_n(pass) * a.Sk), 0, a.Sk, 0x00020000);
        mbn = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rm, moff, 0, 0);
        kopn = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rk, kvoff, 0, 0));
        vopn = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rv, kvoff, 0, 0));
    };

    float dbias[HT][8];
    if constexpr (DBIAS) {
#pragma unroll
        for (int u = 0; u < HT; ++u)
#pragma unroll
            for (int j = 0; j < 8; ++j) dbias[u][j] = 0.f;
    }

    if (rows > 0) {
        fetch_kv(0);
        fetch_s(0, 0);
        stage(0);
        fetch_s(1 / kSteps, 1 % kSteps);
    }
    __syncthreads();

    for (int pass = 0; pass < rows; ++pass) {
        const int n = n_begin + pass;
        const bool alive = kin && mbn != 0u;
        const half8 kop = alive && a.kscale ? kopn : bzero8();
        const half8 vop = alive ? vopn : bzero8();
        // a dead key's lane: the masked-logit bias row, and -delta from the zeroed area
        const float* const brow = bias_l + (alive ? klocal : 64) * kBRow + qh * HT * 32 + 8 * g;
        const float* const qtS = qterms + qh * 128 + 8 * g;
        const float* const qtD = qtS + 32 + (alive ? 0 : 512);
        float4v accv[2], acck[2];
#pragma unroll
        for (int db = 0; db < 2; ++db) {
            accv[db] = float4v{0.f, 0.f, 0.f, 0.f};
            acck[db] = float4v{0.f, 0.f, 0.f, 0.f};
        }
        fetch_kv(pass + 1);

#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            const int par = (pass * kSteps + st) & 1;
            // stage the next step (loaded a step ago), fetch the one after it
            stage(par ^ 1);
            fetch_s(pass + (st + 2) / kSteps, (st + 2) % kSteps);
            const half_t* buf = lds + par * kBuf + qh * 2 * kSub;
            // the step's two tiles phase by phase, so each phase has two independent chains
            float x[2][8];
            float4v dp[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int u = 2 * st + i;
                const half_t* Qs = buf + i * kSub;
                const half_t* Os = Qs + kOs;
                const int qo = par * 256 + 64 * i;
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    float4v sacc = *reinterpret_cast<const float4v*>(qtS + qo + 4 * qb);
                    dp[i][qb] = *reinterpret_cast<const float4v*>(qtD + qo + 4 * qb);
                    const int w = 2 * reg_word(16 * qb + r16, 8 * g);
                    const half8 qa = *reinterpret_cast<const half8*>(Qs + w);
                    const half8 oa = *reinterpret_cast<const half8*>(Os + w);
                    sacc = mfma16x16x32(qa, kop, sacc);
                    dp[i][qb] = mfma16x16x32(oa, vop, dp[i][qb]);
                    const float4 bb = *reinterpret_cast<const float4*>(brow + 32 * u + 4 * qb);
                    x[i][4 * qb + 0] = fmaf(sacc[0], c1, bb.x);
                    x[i][4 * qb + 1] = fmaf(sacc[1], c1, bb.y);
                    x[i][4 * qb + 2] = fmaf(sacc[2], c1, bb.z);
                    x[i][4 * qb + 3] = fmaf(sacc[3], c1, bb.w);
                }
            }
            half8 pb[2], dsb[2];
            float dsf[2][8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const float p = exp2_fast(x[i][j]);
                    dsf[i][j] = pin_f32(p * dp[i][j >> 2][j & 3]);
                    pb[i][j] = (half_t)p;
                    dsb[i][j] = (half_t)dsf[i][j];
                }
            if constexpr (DBIAS) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j) dbias[2 * st + i][j] = pin_f32(dbias[2 * st + i][j] + dsf[i][j]);
            }
            // dV^T += dO^T P, dK^T += Q^T dS (k-slots queries 8 g + j, read transposed)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const half_t* Qs = buf + i * kSub;
                const half_t* Os = Qs + kOs;
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    const half8 ot = reg_operand_tr(Os, g, r16, db);
                    const half8 qt = reg_operand_tr(Qs, g, r16, db);
                    accv[db] = mfma16x16x32(ot, pb[i], accv[db]);
                    acck[db] = mfma16x16x32(qt, dsb[i], acck[db]);
                }
            }
            if (st == kSteps - 1 && qh == 1) {
                // this half's sums of the row, for the half 0 wave of the same keys
                float4* r = red + ((T::kSlots == 2 ? (pass & 1) : 0) * 4 + kg) * 4 * 64 + lane;
                r[0] = make_float4(acck[0][0], acck[0][1], acck[0][2], acck[0][3]);
                r[64] = make_float4(acck[1][0], acck[1][1], acck[1][2], acck[1][3]);
                r[128] = make_float4(accv[0][0], accv[0][1], accv[0][2], accv[0][3]);
                r[192] = make_float4(accv[1][0], accv[1][1], accv[1][2], accv[1][3]);
            }
            __syncthreads();
        }

        if (qh == 0 && kin) {
            // half 0 + half 1, then lane holds d = 8 g .. + 8 of its key (a masked key's dS,
            // and so dK, is 0)
            const float4* r = red + ((T::kSlots == 2 ? (pass & 1) : 0) * 4 + kg) * 4 * 64 + lane;
            const float4 k0 = r[0], k1 = r[64], v0 = r[128], v1 = r[192];
            const float ks[8] = {acck[0][0] + k0.x, acck[0][1] + k0.y, acck[0][2] + k0.z, acck[0][3] + k0.w,
                                 acck[1][0] + k1.x, acck[1][1] + k1.y, acck[1][2] + k1.z, acck[1][3] + k1.w};
            const float vs[8] = {accv[0][0] + v0.x, accv[0][1] + v0.y, accv[0][2] + v0.z, accv[0][3] + v0.w,
                                 accv[1][0] + v1.x, accv[1][1] + v1.y, accv[1][2] + v1.z, accv[1][3] + v1.w};
            const int64_t off = (((int64_t)n * a.H + h) * a.Sk + key) * DP + 8 * g;
            half8 ok, ov;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                ok[j] = (half_t)(ks[j] * a.scale);
                ov[j] = (half_t)vs[j];
            }
            *reinterpret_cast<half8*>(a.dk + off) = ok;
            *reinterpret_cast<half8*>(a.dv + off) = ov;
        }
    }

    if constexpr (DBIAS) {
        // the chunk's [SqA][64] partial: query 32 (qh HT + u) + 8 g + j, this lane's key column
        const int qtiles = a.SqA / 32;
        float* dst = a.partial + (((int64_t)c * a.H + h) * a.kblocks + kblk) * a.SqA * 64 + klocal;
#pragma unroll
        for (int u = 0; u < HT; ++u) {
            const int ut = qh * HT + u;
            if (ut >= qtiles) continue;
#pragma unroll
            for (int j = 0; j < 8; ++j) dst[(int64_t)(32 * ut + 8 * g + j) * 64] = dbias[u][j];
        }
    }
}

// ------------------------------------------------------------------------------------------
// The register dK/dV kernel in query parts, D = 32: for QT = 12 (256 < Sq <= 384) twelve waves
// at three per SIMD, key group w % 4 by query third w / 4 (four tiles each, two per step), so the
// dBias partial is 32 registers per lane and the kernel fits 168 VGPRs; for QT = 8 (128 < Sq <=
// 256) sixteen waves at four per SIMD, key group w % 4 by query quarter w / 4 (two tiles each, one
// per step), 16 registers of partial within 128 VGPRs. Its LDS holds the workgroup's bias as
// fp16 (the original values, recovered exactly from the fp32 log2e form), so s2 = log2e (scale S
// + bias) takes an fma with the fp16 operand read in place and a multiply. The parts' dK / dV
// sums meet in LDS once per row, parts 1, 2 (, 3) into part 0 in that order.
// The Q / dO tiles and the query terms of the next step go straight from memory into the idle
// LDS buffer by direct-to-LDS loads (buffer_load ... lds), issued at the start of a step and
// complete at its closing barrier: no staging registers and no LDS store instructions. The two
// buffers (and the two term buffers) are separate arrays with compile-time selection, so the
// compiler can tell that the step's LDS reads do not alias the loads in flight and does not wait
// for them. Everything else is attn_bwd_dkdv_reg_kernel's.
// ------------------------------------------------------------------------------------------
template <int QT>
struct PartTile {
    static constexpr int kParts = QT == 12 ? 3 : 4;      // query parts (waves per key group)
    static constexpr int kThreads = 4 * kParts * kWave;
    static constexpr int kTPS = QT == 12 ? 2 : 1;        // tiles per part and step
};

template <int QT, bool DBIAS>
__global__ __launch_bounds__(PartTile<QT>::kThreads, QT == 12 ? 3 : 4) void attn_bwd_dkdv_reg3_kernel(BwdArgs a) {
    static_assert(QT == 12 || QT == 8, "query parts of two tiles per step (QT 12) or one (QT 8)");
    constexpr int kParts = PartTile<QT>::kParts, kTPS = PartTile<QT>::kTPS, kNT = PartTile<QT>::kThreads;
    constexpr int DP = 32, TT = QT / kParts;  // tiles per part
    constexpr int kSteps = TT / kTPS;
    static_assert(kSteps == 2, "buffer parity alternates by step within a row");
    constexpr int kTile = 32 * DP, kOs = kTile + 64, kSub = kOs + kTile;
    constexpr int kBuf = kParts * kTPS * kSub;  // halfs of a step: [part][tile]
    constexpr int kQTerms = kParts * kTPS * 16; // float4 slots of a step's query terms
    constexpr int SqB = 32 * QT;
    constexpr int kBRow = SqB + 8;           // LDS bias row stride (halfs)
    __shared__ __attribute__((aligned(16))) half_t bias_l[65 * kBRow];  // rows: 64 keys, masked
    __shared__ __attribute__((aligned(16))) half_t lds0[kBuf];
    __shared__ __attribute__((aligned(16))) half_t lds1[kBuf];
    // query terms of each buffer [part][tile][-lse2 / c1 x 32, -delta x 32] (at most 384 of the
    // first 512 floats), then 384 zeros, the -delta a dead key's lane reads
    __shared__ __attribute__((aligned(16))) float qterms0[512 + 384];
    __shared__ __attribute__((aligned(16))) float qterms1[512 + 384];
    // parts 1 .. kParts - 1's dK / dV sums of a row: [part - 1][key group][float4 j][lane]
    __shared__ __attribute__((aligned(16))) float4 red[(kParts - 1) * 4 * 4 * 64];

    const int item = xcd_item(blockIdx.x, gridDim.x);
    const int rest = fdiv(item, a.fkb), kblk = item - rest * a.kblocks;
    const int h = fdiv(rest, a.fch), c = rest - h * a.chunks;
    const int n_begin = c * a.chunk;
    const int rows = min(a.N, n_begin + a.chunk) - n_begin;
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int kg = wave & 3, q3 = wave >> 2;  // key group, query part
    const int r16 = lane & 15, g = lane >> 4;
    const int klocal = kg * 16 + r16;
    const int key = kblk * 64 + klocal;
    const bool kin = key < a.Sk;
    const float c1s = a.c1s;

    if (tid < 192) reinterpret_cast<float4*>(tid < 96 ? qterms0 + 512 : qterms1 + 128)[tid] = make_float4(0.f, 0.f, 0.f, 0.f);

    // this wave's staging share of a step: tile (part sq3, tile si) of tensor (Q, dO); waves past
    // the step's kParts kTPS tiles x 2 tensors stage none
    const int ti = wave >> 1, tensor = wave & 1, sq3 = ti / kTPS, si = ti % kTPS;
    const bool stager = 2 * kTPS >= 4 || wave < 2 * kParts * kTPS;
    // as two direct-to-LDS loads of 16 LDS rows each: slot l of load i is LDS row R = 16 i + l / 4,
    // position p = l % 4, which holds chunk p ^ ((R / 4) % 4) of tile row x (perm_row(x, 8) = R)
    uint32_t dvoff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int R = 16 * i + (lane >> 2), p = lane & 3;
        const int x = 8 * ((R >> 2) & 3) + 4 * (R >> 4) + (R & 3);
        dvoff[i] = (uint32_t)((x * DP + 8 * (p ^ ((R >> 2) & 3))) * 2);
    }
    const int dst_off = (kTPS * sq3 + si) * kSub + tensor * kOs;
    const half_t* const csrc = tensor ? a.dout : a.q;
    // the first waves stage the query terms: flat lane L < kQTerms, tile L / 16 of [part][tile]
    const int qL = wave * kWave + lane;
    const int qt_t = qL >> 4;
    const uint32_t qt_f = (uint32_t)(4 * (qL & 15));

    const auto row_n = [&](int pass) -> int { return n_begin + (pass < rows ? pass : 0); };
    const auto row_nh = [&](int pass) -> int64_t { return (int64_t)row_n(pass) * a.H + h; };
    // step `step` of row `pass` into LDS buffer buf, by direct-to-LDS loads: this wave's tile, and
    // (the first waves) the step's query terms, lane qL to float 4 qL of the buffer's terms (lanes
    // past kQTerms write zeros into its unused tail)
    const auto dma_s = [&](int pass, int step, int buf) {
        const int64_t nh = row_nh(pass);
        if (stager) {
            const int q0 = 32 * (sq3 * TT + kTPS * step + si);
            const auto rs = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<half_t*>(csrc + (nh * a.Sq + q0) * DP), 0, max(a.Sq - q0, 0) * DP * 2, 0x00020000);
            half_t* dst = (buf ? lds1 : lds0) + dst_off;
#pragma unroll
            for (int i = 0; i < 2; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rs, (__attribute__((address_space(3))) void*)(dst + 512 * i), 16, dvoff[i], 0, 0, 0);
        }
        if (wave * kWave < kQTerms) {
            const int tg = (qt_t / kTPS) * TT + kTPS * step + (qt_t % kTPS);
            const auto rq = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(a.qstat + nh * a.SqA * 2), 0, a.SqA * 2 * 4, 0x00020000);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rq, (__attribute__((address_space(3))) void*)((buf ? qterms1 : qterms0) + 256 * wave), 16,
                qL < kQTerms ? ((uint32_t)(64 * tg) + qt_f) * 4u : 0x80000000u, 0, 0, 0);
        }
    };

    // the lane's K/V chunk and mask byte of a row: buffer loads from the row's (scalar) base at
    // offsets fixed for the kernel
    half8 kopn, vopn;
    uint32_t mbn = 0u;
    const uint32_t kvoff = (uint32_t)((kin ? key : 0) * DP + 8 * g) * 2u, moff = (uint32_t)(kin ? key : 0);
    const auto fetch_kv = [&](int pass) {
        const int64_t nh = row_nh(pass);
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.k + nh * a.Sk * DP), 0, a.Sk * DP * 2, 0x00020000);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.v + nh * a.Sk * DP), 0, a.Sk * DP * 2, 0x00020000);
        const auto rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.kmask + (int64_t)row_n(pass) * a.Sk), 0, a.Sk, 0x00020000);
        mbn = (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rm, moff, 0, 0);
        kopn = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rk, kvoff, 0, 0));
        vopn = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rv, kvoff, 0, 0));
    };

    float dbias[TT][8];
    if constexpr (DBIAS) {
#pragma unroll
        for (int u = 0; u < TT; ++u)
#pragma unroll
            for (int j = 0; j < 8; ++j) dbias[u][j] = 0.f;
    }

    if (rows > 0) {
        fetch_kv(0);
        dma_s(0, 0, 0);
    }
    // (after the first step's loads are issued, so that their latency and the bias loads' overlap)
    // the workgroup's bias, fp16: rows kblk 64 .. + 63 and the masked-logit row SkA
    {
        constexpr int kFill = (65 * (SqB / 4) + kNT - 1) / kNT;
        const float* src = a.biast + (int64_t)h * (a.SkA + 1) * SqB;
#pragma unroll
        for (int f = 0; f < kFill; ++f) {
            const int idx = tid + kNT * f;
            if (idx < 65 * (SqB / 4)) {
                const int r = idx / (SqB / 4), c4 = idx - r * (SqB / 4);
                const int srow = r < 64 ? kblk * 64 + r : a.SkA;
                const float4 v = *reinterpret_cast<const float4*>(src + (int64_t)srow * SqB + 4 * c4);
                *reinterpret_cast<half4*>(bias_l + r * kBRow + 4 * c4) =
                    half4{(half_t)(v.x * (1.f / kLog2e)), (half_t)(v.y * (1.f / kLog2e)),
                          (half_t)(v.z * (1.f / kLog2e)), (half_t)(v.w * (1.f / kLog2e))};
            }
        }
    }
    __syncthreads();

    for (int pass = 0; pass < rows; ++pass) {
        const int n = n_begin + pass;
        const bool alive = kin && mbn != 0u;
        const half8 kop = alive && a.kscale ? kopn : bzero8();
        const half8 vop = alive ? vopn : bzero8();
        // a dead key's lane: the masked-logit bias row, and -delta from the zeroed area
        const half_t* const brow = bias_l + (alive ? klocal : 64) * kBRow + q3 * TT * 32 + 8 * g;
        const int qtS = q3 * kTPS * 64 + 8 * g;
        const int qtD = qtS + 32 + (alive ? 0 : 512);
        float4v accv[2], acck[2];
#pragma unroll
        for (int db = 0; db < 2; ++db) {
            accv[db] = float4v{0.f, 0.f, 0.f, 0.f};
            acck[db] = float4v{0.f, 0.f, 0.f, 0.f};
        }
        fetch_kv(pass + 1);

#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            const int par = st & 1;  // kSteps is even
            // the next step's tiles into the other buffer, whose last reads ended at the barrier
            dma_s(pass + (st + 1) / kSteps, (st + 1) % kSteps, par ^ 1);
            const half_t* buf = (par ? lds1 : lds0) + q3 * kTPS * kSub;
            const float* qtb = par ? qterms1 : qterms0;
            // The step's two tiles as a pipeline: tile 1's S and dP products run beside tile 0's
            // softmax, and tile 0's dV / dK products beside tile 1's, so that each wave has
            // matrix-core work in flight while it issues vector instructions.
            float4v sacc[kTPS][2], dp[kTPS][2];
            half8 bb[kTPS], pb[kTPS], dsb[kTPS];
            // S and dP of tile i: the LDS reads and four MFMAs
            const auto sdp = [&](int i) __attribute__((always_inline)) {
                const int u = kTPS * st + i;
                const half_t* Qs = buf + i * kSub;
                const half_t* Os = Qs + kOs;
                const int qo = 64 * i;
                bb[i] = *reinterpret_cast<const half8*>(brow + 32 * u);
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    sacc[i][qb] = *reinterpret_cast<const float4v*>(qtb + qtS + qo + 4 * qb);
                    dp[i][qb] = *reinterpret_cast<const float4v*>(qtb + qtD + qo + 4 * qb);
                    const int w = 2 * reg_word(16 * qb + r16, 8 * g);
                    const half8 qa = *reinterpret_cast<const half8*>(Qs + w);
                    const half8 oa = *reinterpret_cast<const half8*>(Os + w);
                    sacc[i][qb] = mfma16x16x32(qa, kop, sacc[i][qb]);
                    dp[i][qb] = mfma16x16x32(oa, vop, dp[i][qb]);
                }
            };
            // the softmax of tile i: s2 = log2e (scale S + bias), p, dS = p dP, their fp16
            // operands and the dBias adds
            const auto soft = [&](int i) __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float x = fmaf(sacc[i][j >> 2][j & 3], c1s, (float)bb[i][j]) * kLog2e;
                    const float p = exp2_fast(x);
                    const float dsf = pin_f32(p * dp[i][j >> 2][j & 3]);
                    pb[i][j] = (half_t)p;
                    dsb[i][j] = (half_t)dsf;
                    if constexpr (DBIAS) dbias[kTPS * st + i][j] = pin_f32(dbias[kTPS * st + i][j] + dsf);
                }
            };
            // dV^T += dO^T P and dK^T += Q^T dS of tile i (k-slots queries 8 g + j, read transposed)
            const auto dvdk = [&](int i) __attribute__((always_inline)) {
                const half_t* Qs = buf + i * kSub;
                const half_t* Os = Qs + kOs;
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    const half8 ot = reg_operand_tr(Os, g, r16, db);
                    const half8 qt = reg_operand_tr(Qs, g, r16, db);
                    accv[db] = mfma16x16x32(ot, pb[i], accv[db]);
                    acck[db] = mfma16x16x32(qt, dsb[i], acck[db]);
                }
            };
            if constexpr (kTPS == 2) {
                sdp(0);
                sdp(1);
                soft(0);
                dvdk(0);
                soft(1);
                dvdk(1);
            } else {
                sdp(0);
                soft(0);
                dvdk(0);
            }
#ifdef CLK_REG3_SGB
            // tile 0's reads and products; tile 1's reads; tile 1's products each beside a quarter
            // of tile 0's softmax; tile 0's transposed reads; its dV / dK products each beside a
            // quarter of tile 1's softmax; tile 1's transposed reads and products
            __builtin_amdgcn_sched_group_barrier(0x100, 9, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 9, 0);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
#endif
            if (st == kSteps - 1 && q3 > 0) {
                float4* r = red + ((q3 - 1) * 4 + kg) * 4 * 64 + lane;
                r[0] = make_float4(acck[0][0], acck[0][1], acck[0][2], acck[0][3]);
                r[64] = make_float4(acck[1][0], acck[1][1], acck[1][2], acck[1][3]);
                r[128] = make_float4(accv[0][0], accv[0][1], accv[0][2], accv[0][3]);
                r[192] = make_float4(accv[1][0], accv[1][1], accv[1][2], accv[1][3]);
            }
            // the next step's tiles and terms, loaded straight into LDS at the start of this
            // step, have landed before the barrier after which every wave reads them (the
            // compiler also waits for all loads before a barrier; the order does not rest on it)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }

        if (q3 == 0 && kin) {
            // part 0 + part 1 + ..., then lane holds d = 8 g .. + 8 of its key
            float ks[8], vs[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                ks[j] = acck[j / 4][j & 3];
                vs[j] = accv[j / 4][j & 3];
            }
#pragma unroll
            for (int t = 0; t < kParts - 1; ++t) {
                const float4* r = red + (t * 4 + kg) * 4 * 64 + lane;
                const float4 k0 = r[0], k1 = r[64], v0 = r[128], v1 = r[192];
                ks[0] += k0.x; ks[1] += k0.y; ks[2] += k0.z; ks[3] += k0.w;
                ks[4] += k1.x; ks[5] += k1.y; ks[6] += k1.z; ks[7] += k1.w;
                vs[0] += v0.x; vs[1] += v0.y; vs[2] += v0.z; vs[3] += v0.w;
                vs[4] += v1.x; vs[5] += v1.y; vs[6] += v1.z; vs[7] += v1.w;
            }
            const int64_t off = (((int64_t)n * a.H + h) * a.Sk + key) * DP + 8 * g;
            half8 ok, ov;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                ok[j] = (half_t)(ks[j] * a.scale);
                ov[j] = (half_t)vs[j];
            }
            *reinterpret_cast<half8*>(a.dk + off) = ok;
            *reinterpret_cast<half8*>(a.dv + off) = ov;
        }
    }

    if constexpr (DBIAS) {
        const int qtiles = a.SqA / 32;
        float* dst = a.partial + (((int64_t)c * a.H + h) * a.kblocks + kblk) * a.SqA * 64 + klocal;
#pragma unroll
        for (int u = 0; u < TT; ++u) {
            const int ut = q3 * TT + u;
            if (ut >= qtiles) continue;
#pragma unroll
            for (int j = 0; j < 8; ++j) dst[(int64_t)(32 * ut + 8 * g + j) * 64] = dbias[u][j];
        }
    }
}

template __global__ void attn_bwd_dkdv_reg3_kernel<12, true>(BwdArgs);
template __global__ void attn_bwd_dkdv_reg3_kernel<12, false>(BwdArgs);
template __global__ void attn_bwd_dkdv_reg3_kernel<8, true>(BwdArgs);
template __global__ void attn_bwd_dkdv_reg3_kernel<8, false>(BwdArgs);

// With more than one query window: dk = fp16(scale * sum of the windows' dK sums), dv = fp16(sum
// of their dV sums), each summed in window order, four elements per thread (D % 4 == 0).
__global__ __launch_bounds__(256) void attn_bwd_dkdv_sum_kernel(BwdArgs a) {
    const int64_t plane = (int64_t)a.N * a.H * a.Sk * a.D;
    for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < plane;
         i += (int64_t)gridDim.x * blockDim.x * 4) {
        float4 sk = *reinterpret_cast<const float4*>(a.dkv + i);
        float4 sv = *reinterpret_cast<const float4*>(a.dkv + a.windows * plane + i);
        for (int w = 1; w < a.windows; ++w) {
            const float4 k = *reinterpret_cast<const float4*>(a.dkv + w * plane + i);
            const float4 v = *reinterpret_cast<const float4*>(a.dkv + (a.windows + w) * plane + i);
            sk.x += k.x; sk.y += k.y; sk.z += k.z; sk.w += k.w;
            sv.x += v.x; sv.y += v.y; sv.z += v.z; sv.w += v.w;
        }
        half4 ok = half4{(half_t)(sk.x * a.scale), (half_t)(sk.y * a.scale), (half_t)(sk.z * a.scale),
                         (half_t)(sk.w * a.scale)};
        half4 ov = half4{(half_t)sv.x, (half_t)sv.y, (half_t)sv.z, (half_t)sv.w};
        *reinterpret_cast<half4*>(a.dk + i) = ok;
        *reinterpret_cast<half4*>(a.dv + i) = ov;
    }
}

// biast[h][key][q] = log2e bias[h][q][key] in fp32 for q < Sq, key < Sk, else -inf, over
// [H][SkA + 1][SqB]: a workgroup transposes 32 queries x 64 keys through LDS, with 16-byte loads
// where the bias rows allow them and 16-byte stores (SqB is a multiple of 32). The workgroups of
// key block 0 also write their queries of row SkA: log2e kMaskedLogit (q < Sq), else -inf.
__global__ __launch_bounds__(256) void attn_bwd_biast_kernel(BwdArgs a) {
    __shared__ half_t tile[32][66];
    const int qtiles = a.SqB / 32;
    const int item = blockIdx.x;
    const int qt = item % qtiles, rest = item / qtiles;
    const int kblk = rest % a.kblocks, h = rest / a.kblocks;
    const int tid = threadIdx.x;
    const int q0 = qt * 32, k0 = kblk * 64;
    {
        const int qq = tid / 8, kc = (tid % 8) * 8;
        const int gq = q0 + qq;
        const int valid = gq < a.Sq ? a.Sk - (k0 + kc) : 0;
        const half_t* src = a.bias + ((int64_t)h * a.Sq + (gq < a.Sq ? gq : 0)) * a.Sk + k0 + kc;
        half8 b;
        if (a.bias_vec && valid >= 8) {
            b = bld8(src);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) b[j] = j < valid ? src[j] : (half_t)0.f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) tile[qq][kc + j] = b[j];
    }
    __syncthreads();
    {
        const int kk = tid / 4, qc = (tid % 4) * 8;
        float8v o;
        const bool kok = k0 + kk < a.Sk;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            o[j] = kok && q0 + qc + j < a.Sq ? (float)tile[qc + j][kk] * kLog2e : -INFINITY;
        }
        *reinterpret_cast<float8v*>(a.biast + ((int64_t)h * (a.SkA + 1) + k0 + kk) * a.SqB + q0 + qc) = o;
        if (kblk == 0 && tid < 32) {
            a.biast[((int64_t)h * (a.SkA + 1) + a.SkA) * a.SqB + q0 + tid] =
                q0 + tid < a.Sq ? kMaskedLogit2 : -INFINITY;
        }
    }
    {
        // the dQ kernel's fragments of this tile's two 16-query blocks: thread t writes block
        // t / 128, part (t / 64) % 2, lane l = t % 64 (query l % 16, keys 16 (l / 16) + 8 part ..)
        const int qb = tid >> 7, part = (tid >> 6) & 1, l = tid & 63;
        const int qblk = q0 / 16 + qb;
        if (qblk < a.SqA / 16) {
            half8 f;
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = tile[16 * qb + (l & 15)][16 * (l >> 4) + 8 * part + j];
            *reinterpret_cast<half8*>(a.bfrag + ((((int64_t)h * (a.SqA / 16) + qblk) * a.kblocks + kblk) * 2 + part) * 512 + 8 * l) = f;
        }
    }
}

// dbias[h][q][key] = the chunks' partials summed in chunk order. A workgroup takes 16 queries x
// 64 keys of one head, a thread four keys of one query; its chunk loads are issued eight at a
// time ahead of their adds, so many are in flight per thread.
__global__ __launch_bounds__(256) void attn_bwd_dbias_kernel(BwdArgs a) {
    const int qgroups = a.SqA / 16;
    const int item = blockIdx.x;
    const int qgrp = item % qgroups, rest = item / qgroups;
    const int kblk = rest % a.kblocks, h = rest / a.kblocks;
    const int k4 = (threadIdx.x & 15) * 4, q = qgrp * 16 + (threadIdx.x >> 4);
    const int64_t stride = (int64_t)a.H * a.kblocks * a.SqA * 64;
    const float* src = a.partial + (((int64_t)h * a.kblocks + kblk) * a.SqA + q) * 64 + k4;
    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
    int c = 0;
    for (; c + 8 <= a.chunks; c += 8) {
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = *reinterpret_cast<const float4*>(src + (c + j) * stride);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sum.x += v[j].x;
            sum.y += v[j].y;
            sum.z += v[j].z;
            sum.w += v[j].w;
        }
    }
    for (; c < a.chunks; ++c) {
        const float4 v = *reinterpret_cast<const float4*>(src + c * stride);
        sum.x += v.x;
        sum.y += v.y;
        sum.z += v.z;
        sum.w += v.w;
    }
    if (q >= a.Sq) return;
    const int key = kblk * 64 + k4;
    float* dst = a.dbias + ((int64_t)h * a.Sq + q) * a.Sk + key;
    if (a.dbias_vec && key + 4 <= a.Sk) {
        *reinterpret_cast<float4*>(dst) = sum;
    } else {
        const float v[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (key + j < a.Sk) dst[j] = v[j];
        }
    }
}

__global__ void fill_zero_f32(float* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        p[i] = 0.f;
    }
}

// ---- host side ----------------------------------------------------------------------------

static int cu_count(int device) {
    static int cache[16] = {};
    if (device < 0 || device >= 16) return 256;
    if (cache[device] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
            v <= 0) {
            v = 256;
        }
        cache[device] = v;
    }
    return cache[device];
}

struct BwdPlan {
    int DP = 32;
    int QT = 0;  // query tiles of the register-partial dK/dV kernel (4, 8 or 12), 0: not used
    int QG = 1;  // query groups of the dK/dV kernel
    int kblocks = 0, chunk = 0, chunks = 0;
    int wtiles = 1, windows = 1;  // query windows of the dK/dV kernel
    size_t stage_lds = 0, dbias_lds = 0;
    int SqA = 0, SkA = 0, SqB = 0;
    size_t delta_bytes = 0, biast_bytes = 0, partial_bytes = 0, dkv_bytes = 0, bfrag_bytes = 0;
    std::string error;
};

static size_t round256(size_t b) { return (b + 255) & ~size_t(255); }

static size_t dkdv_stage_bytes(int DP, int QG) {
#define CLK_STAGE(D_, Q_) if (DP == D_ && QG == Q_) return DkdvTile<D_, Q_>::kStageBytes;
    CLK_STAGE(32, 4) CLK_STAGE(32, 2) CLK_STAGE(32, 1) CLK_STAGE(64, 2) CLK_STAGE(64, 1)
    CLK_STAGE(96, 2) CLK_STAGE(96, 1)
#undef CLK_STAGE
    return 0;
}

// The dK/dV kernel's shape depends only on the problem and the device, never on want_dbias, so
// dk and dv are bit-identical with and without dbias.
//
// Its dBias partial stays in LDS for a whole chunk of rows: 64 keys x the queries of a query
// window, 8 KB per 32-query tile. Where all of Sq does not fit next to the Q/dO staging, the
// queries are split into windows of equal tile counts (one more grid dimension); each window's
// dK and dV sums then go to the workspace in fp32 and dkdv_sum_kernel adds them in window order.
static BwdPlan plan_bwd(int device, int64_t N, int64_t H, int64_t Sq, int64_t Sk, int64_t D) {
    BwdPlan p;
    p.DP = D <= 32 ? 32 : D <= 64 ? 64 : 96;
    p.SqA = (int)(((Sq + 31) / 32) * 32);
    p.kblocks = (int)((Sk + 63) / 64);
    p.SkA = p.kblocks * 64;
    int limit = shared_limit(device);
    if (limit <= 0) limit = 64 * 1024;
    const size_t tile_bytes = (size_t)64 * 32 * sizeof(float);
    const int64_t qtiles = std::max<int64_t>((Sq + 31) / 32, 1);
    const int64_t Nr = std::max<int64_t>(N, 1);  // N == 0 plans one (empty) chunk
    if (D == 32 && qtiles <= 12) {
        // the register-partial kernels: one workgroup of eight (QT 4), sixteen (QT 8) or twelve (QT 12) waves
        // per CU, one row per pass;
        // chunks trade rounds of workgroups against dbias partials to write and sum (one
        // partial weighs about H kblocks / 128 row passes)
        p.QT = qtiles <= 4 ? 4 : qtiles <= 8 ? 8 : 12;
        p.QG = 1;
        p.wtiles = (int)qtiles;
        p.windows = 1;
        const int64_t slots = (int64_t)cu_count(device);
        const int64_t cols = std::max<int64_t>(H * p.kblocks, 1);
        int64_t best = 1;
        double best_cost = 1e300;
        for (int64_t ch = 1; ch <= Nr; ++ch) {
            const int64_t rows = (Nr + ch - 1) / ch;
            const int64_t real = (Nr + rows - 1) / rows;
            const int64_t rounds = (real * cols + slots - 1) / slots;
            const double cost = (double)rounds * rows + (double)real * cols / 128.0;
            if (cost < best_cost) {
                best_cost = cost;
                best = real;
            }
        }
        p.chunk = (int)((Nr + best - 1) / best);
        p.chunks = (int)((N + p.chunk - 1) / p.chunk);
        p.delta_bytes = round256((size_t)N * H * p.SqA * sizeof(float));
        p.SqB = 32 * p.QT;
        p.biast_bytes = round256((size_t)H * (p.SkA + 1) * p.SqB * sizeof(float));
        p.partial_bytes = round256((size_t)p.chunks * H * p.kblocks * p.SqA * 64 * sizeof(float));
        p.bfrag_bytes = round256((size_t)H * p.SqA * p.SkA * sizeof(half_t));
        return p;
    }
    // row groups of the dK/dV kernel: at most the query tiles of a window, which they walk from
    // staggered starts; the most row groups (waves per CU) first, then the fewest windows
    int qg_max = p.DP == 32 ? 4 : 2;
    while (qg_max > qtiles) qg_max /= 2;
    p.QG = 0;
    for (int qg = qg_max; qg >= 1 && p.QG == 0; qg /= 2) {
        const size_t stage = dkdv_stage_bytes(p.DP, qg);
        if (stage + tile_bytes * qg > (size_t)limit) continue;
        const int64_t wmax = (int64_t)((limit - stage) / tile_bytes);
        const int64_t windows = (qtiles + wmax - 1) / wmax;
        const int64_t wtiles = (qtiles + windows - 1) / windows;
        const int64_t last = qtiles - (windows - 1) * wtiles;
        if (last < qg) continue;  // every window needs a tile per row group
        p.QG = qg;
        p.windows = (int)windows;
        p.wtiles = (int)wtiles;
    }
    if (p.QG == 0) {
        p.QG = 1;
        p.windows = (int)qtiles;
        p.wtiles = 1;
        const size_t need = dkdv_stage_bytes(p.DP, 1) + tile_bytes;
        p.error = "attention_bwd: dbias needs " + std::to_string(need / 1024) +
                  " KB shared, device allows " + std::to_string(limit / 1024) + " KB";
    }
    p.stage_lds = dkdv_stage_bytes(p.DP, p.QG);
    p.dbias_lds = tile_bytes * p.wtiles;
    // batch-row chunks: the fewest rounds of workgroups times rows per workgroup
    const size_t per_wg = p.stage_lds + p.dbias_lds;
    const int threads = 256 * p.QG;
    int per_cu = std::max(1, std::min(2048 / threads, (int)(limit / per_wg)));
    const int64_t slots = (int64_t)cu_count(device) * per_cu;
    const int64_t cols = std::max<int64_t>(H * p.kblocks * p.windows, 1);
    int64_t best = 1, best_cost = INT64_MAX;
    for (int64_t ch = 1; ch <= Nr; ++ch) {
        // rows per workgroup, a whole number of passes of its QG row groups where N allows
        const int64_t rows = std::min<int64_t>(((Nr + ch - 1) / ch + p.QG - 1) / p.QG * p.QG, Nr);
        const int64_t real = (Nr + rows - 1) / rows;
        const int64_t rounds = (real * cols + slots - 1) / slots;
        const int64_t passes = (rows + p.QG - 1) / p.QG;
        // each extra chunk adds a dbias partial to write and sum; a pass of the row groups costs
        // about 24 of them per row group
        const int64_t cost = rounds * passes * p.QG * 24 + real;
        if (cost < best_cost) {
            best_cost = cost;
            best = real;
        }
    }
    p.chunk = (int)((Nr + best - 1) / best);
    p.chunks = (int)((N + p.chunk - 1) / p.chunk);
    p.delta_bytes = round256((size_t)N * H * p.SqA * sizeof(float));  // half of the query terms
    p.SqB = p.SqA;
    p.biast_bytes = round256((size_t)H * (p.SkA + 1) * p.SqB * sizeof(float));
    p.partial_bytes = round256((size_t)p.chunks * H * p.kblocks * p.SqA * 64 * sizeof(float));
    p.dkv_bytes = p.windows > 1 ? round256((size_t)2 * p.windows * N * H * Sk * D * sizeof(float)) : 0;
    p.bfrag_bytes = round256((size_t)H * p.SqA * p.SkA * sizeof(half_t));
    return p;
}

static size_t bwd_workspace_bytes(const BwdPlan& p) {
    return 2 * p.delta_bytes + p.biast_bytes + p.partial_bytes + p.dkv_bytes + p.bfrag_bytes;
}

template <int DP, int QG>
static void launch_dkdv(hipStream_t stream, const BwdArgs& a, const BwdPlan& p, bool want_dbias) {
    using T = DkdvTile<DP, QG>;
    const int64_t g2 = (int64_t)p.chunks * a.H * p.kblocks * p.windows;
    const size_t lds = p.stage_lds + (want_dbias ? p.dbias_lds : 0);
    const void* fn = want_dbias ? reinterpret_cast<const void*>(&attn_bwd_dkdv_kernel<DP, QG, true>)
                                : reinterpret_cast<const void*>(&attn_bwd_dkdv_kernel<DP, QG, false>);
    if (lds > 64 * 1024) {
        // LDS past 64 KB per workgroup is opt-in on some runtimes; a failure shows at launch
        (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    }
    if (want_dbias) {
        hipLaunchKernelGGL((attn_bwd_dkdv_kernel<DP, QG, true>), dim3((unsigned)g2), dim3(T::kThreads),
                           lds, stream, a);
    } else {
        hipLaunchKernelGGL((attn_bwd_dkdv_kernel<DP, QG, false>), dim3((unsigned)g2), dim3(T::kThreads),
                           lds, stream, a);
    }
}

template <int DP>
static int launch_bwd(hipStream_t stream, const BwdArgs& a, const BwdPlan& p, bool want_dbias) {
    using Q = DqTile<DP>;
    const int64_t qt = (a.Sq + Q::kBQ - 1) / Q::kBQ;
    const int64_t g1 = qt * a.H * a.N;
    if (g1 > INT32_MAX) return invalid("attention_bwd: too many work items");
    stage_mark(stream, 0);
    const int64_t gb = (int64_t)(a.SqB / 32) * p.kblocks * a.H;
    hipLaunchKernelGGL(attn_bwd_biast_kernel, dim3((unsigned)gb), dim3(256), 0, stream, a);
    stage_mark(stream, 1);
    BwdArgs aq = a;
    aq.fqt = fast_div(qt);  // the dQ kernel's query tiles per (n, h), at its DP's tile height
    hipLaunchKernelGGL(attn_bwd_dq_kernel<DP>, dim3((unsigned)g1), dim3(Q::kThreads), 0, stream, aq);
    stage_mark(stream, 2);
    if (p.QT > 0) {
        if constexpr (DP == 32) {
            const int64_t g2 = (int64_t)p.chunks * a.H * p.kblocks;
#define CLK_DKDV_REG(QT_)                                                                        \
    if (p.QT == QT_) {                                                                           \
        if (want_dbias) {                                                                        \
            hipLaunchKernelGGL((attn_bwd_dkdv_reg_kernel<QT_, true>), dim3((unsigned)g2), dim3(512), 0, stream, a); \
        } else {                                                                                 \
            hipLaunchKernelGGL((attn_bwd_dkdv_reg_kernel<QT_, false>), dim3((unsigned)g2), dim3(512), 0, stream, a); \
        }                                                                                        \
    }
            CLK_DKDV_REG(4)
#define CLK_DKDV_PARTS(QT_)                                                                      \
    if (p.QT == QT_) {                                                                           \
        constexpr int kNT = PartTile<QT_>::kThreads;                                             \
        if (want_dbias) {                                                                        \
            hipLaunchKernelGGL((attn_bwd_dkdv_reg3_kernel<QT_, true>), dim3((unsigned)g2), dim3(kNT), 0, stream, a); \
        } else {                                                                                 \
            hipLaunchKernelGGL((attn_bwd_dkdv_reg3_kernel<QT_, false>), dim3((unsigned)g2), dim3(kNT), 0, stream, a); \
        }                                                                                        \
    }
            CLK_DKDV_PARTS(8) CLK_DKDV_PARTS(12)
#undef CLK_DKDV_PARTS
#undef CLK_DKDV_REG
        }
    } else if (p.QG == 4) {
        if constexpr (DP == 32) launch_dkdv<DP, 4>(stream, a, p, want_dbias);
    } else if (p.QG == 2) {
        launch_dkdv<DP, 2>(stream, a, p, want_dbias);
    } else {
        launch_dkdv<DP, 1>(stream, a, p, want_dbias);
    }
    if (p.windows > 1) {
        const int64_t n4 = (int64_t)a.N * a.H * a.Sk * a.D / 4;
        const int64_t gs = std::min<int64_t>((n4 + 255) / 256, 8192);
        hipLaunchKernelGGL(attn_bwd_dkdv_sum_kernel, dim3((unsigned)gs), dim3(256), 0, stream, a);
    }
    stage_mark(stream, 3);
    if (want_dbias) {
        const int64_t g3 = (int64_t)(a.SqA / 16) * p.kblocks * a.H;
        hipLaunchKernelGGL(attn_bwd_dbias_kernel, dim3((unsigned)g3), dim3(256), 0, stream, a);
    } else {
        const int64_t nb = (int64_t)a.H * a.Sq * a.Sk;
        hipLaunchKernelGGL(fill_zero_f32, dim3(1024), dim3(256), 0, stream, a.dbias, nb);
    }
    stage_mark(stream, 4);
    return launch_status("attention_bwd");
}

static bool bwd_head_dim_ok(int64_t d) {
    return d == 8 || d == 16 || d == 24 || d == 32 || d == 48 || d == 64 || d == 96;
}

}  // namespace clk

using namespace clk;

extern "C" size_t clk_attention_bwd_workspace_size(int32_t device, const clk_buffer* q,
                                                   const clk_buffer* k) {
    if (q == nullptr || k == nullptr || q->rank != 4 || k->rank != 4) return 0;
    const BwdPlan p = plan_bwd(device, q->dims[0], q->dims[1], q->dims[2], k->dims[2], q->dims[3]);
    return bwd_workspace_bytes(p);
}

extern "C" int clk_attention_bwd_plan(int32_t device, int64_t N, int64_t H, int64_t Sq,
                                      int64_t Sk, int64_t D, int64_t* plan, int32_t count) {
    if (N < 0 || H < 0 || Sq < 0 || Sk < 0 || !bwd_head_dim_ok(D)) {
        return invalid("attention_bwd_plan: bad shape");
    }
    if (plan == nullptr || count < 0) return invalid("attention_bwd_plan: no output array");
    const BwdPlan p = plan_bwd(device, N, H, Sq, Sk, D);
    const int64_t vals[] = {p.QG, p.chunk, p.chunks, (p.chunk + p.QG - 1) / p.QG, p.windows,
                            p.QT > 0 ? 1 : 0};
    for (int i = 0; i < count && i < 6; ++i) plan[i] = vals[i];
    return ok();
}

// The size of the static scratch of clk_attention_bwd_noalloc: enough for BASELINE C3
// ([512, 8, 384, 32]: 86.3 MiB of query terms, transposed bias and dBias partials).
constexpr size_t kNoAllocScratchBytes = size_t(96) << 20;

// The scratch of clk_attention_bwd_noalloc, one copy per GPU, held until the process ends. Host
// code never uses this name as an address: scratch_address() asks the runtime for each device's
// copy once, with that device current, and every use goes through the pointer it returns.
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

static int scratch_address(int device, void** out) {
    constexpr int kDevices = 16;
    static std::mutex mu;
    static void* ptrs[kDevices] = {};
    if (device < 0 || device >= kDevices) {
        return invalid("attention_bwd_noalloc: device " + std::to_string(device) + " out of range");
    }
    std::lock_guard<std::mutex> lock(mu);
    if (ptrs[device] == nullptr) {
        int cur = -1;
        hipError_t err = hipGetDevice(&cur);
        if (err == hipSuccess && cur != device) err = hipSetDevice(device);
        if (err != hipSuccess) {
            return fail(CLK_INTERNAL, std::string("attention_bwd_noalloc: cannot select device: ") +
                                          hipGetErrorString(err));
        }
        void* p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != device) (void)hipSetDevice(cur);
        if (err != hipSuccess || p == nullptr) {
            return fail(CLK_INTERNAL, std::string("attention_bwd_noalloc: hipGetSymbolAddress: ") +
                                          hipGetErrorString(err));
        }
        ptrs[device] = p;
    }
    *out = ptrs[device];
    return CLK_OK;
}

// clk_attention_bwd, with its workspace given (noalloc false) or taken from the static scratch.
static int attention_bwd_impl(clk_stream stream, int32_t device, const clk_buffer* q,
                              const clk_buffer* k, const clk_buffer* v, const clk_buffer* bias,
                              const clk_buffer* kmask, const clk_buffer* out,
                              const clk_buffer* dout, const clk_buffer* lse, const clk_buffer* dq,
                              const clk_buffer* dk, const clk_buffer* dv, const clk_buffer* dbias,
                              float scale, int32_t want_dbias, void* workspace,
                              size_t workspace_bytes, bool noalloc) {
    const clk_buffer* bufs[] = {q, k, v, bias, kmask, out, dout, lse, dq, dk, dv, dbias};
    const int types[] = {CLK_F16, CLK_F16, CLK_F16, CLK_F16, CLK_U8,  CLK_F16,
                         CLK_F16, CLK_F32, CLK_F16, CLK_F16, CLK_F16, CLK_F32};
    if (int st = check_types("attention_bwd", bufs, types, 12)) return st;
    if (q->rank != 4) return invalid("q must be [N,H,S,D]");
    const int64_t N = q->dims[0], H = q->dims[1], Sq = q->dims[2], D = q->dims[3];
    if (k->rank != 4 || k->dims[0] != N || k->dims[1] != H || k->dims[3] != D) {
        return invalid("volta_mma_bwd: k must be [N,H,Sk,D] like q");
    }
    const int64_t Sk = k->dims[2];
    if (!same_shape(v, k) || !same_shape(dout, q)) {
        return invalid("volta_mma_bwd: v must match k, dout must match q");
    }
    if (!dims_are(lse, N, H, Sq)) return invalid("volta_mma_bwd: lse must be [N,H,Sq]");
    if (!same_shape(out, q)) return invalid("volta_mma_bwd: out must match q");
    if (!dims_are(bias, H, Sq, Sk) || !dims_are(dbias, H, Sq, Sk)) {
        return invalid("volta_mma_bwd: bias and dbias must be [H,Sq,Sk]");
    }
    if (!same_shape(dq, q) || !same_shape(dk, k) || !same_shape(dv, k)) {
        return invalid("volta_mma_bwd: dq, dk, dv must match q, k, v");
    }
    if (elements(kmask) != N * Sk) return invalid("volta_mma_bwd: kmask must be [N,Sk]");
    if (!bwd_head_dim_ok(D)) return invalid("volta_mma_bwd: unsupported head dim");
    const void* vec[] = {q->data, k->data, v->data, out->data, dout->data, dq->data, dk->data, dv->data};
    for (const void* p : vec) {
        if (!aligned16(p)) return invalid("volta_mma_bwd: q, k, v, out, dout, dq, dk, dv must be 16-byte aligned");
    }
    const BwdPlan p = plan_bwd(device, N, H, Sq, Sk, D);
    if (want_dbias && !p.error.empty()) return invalid(p.error);
    if (N * H * Sq == 0 && N * H * Sk == 0 && H * Sq * Sk == 0) return ok();  // nothing to write
    const size_t need = bwd_workspace_bytes(p);
    if (noalloc) {
        if (need > kNoAllocScratchBytes) {
            return invalid("attention_bwd_noalloc: these shapes need " + std::to_string(need) +
                           " bytes of scratch, the library's static scratch holds " +
                           std::to_string(kNoAllocScratchBytes));
        }
        if (int st = scratch_address(device, &workspace)) return st;
        workspace_bytes = kNoAllocScratchBytes;
    }
    if (workspace == nullptr || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255u)) {
        return fail(CLK_INTERNAL, "volta_mma_bwd: the workspace must be 256-byte aligned and hold " +
                                      std::to_string(need) + " bytes");
    }
    BwdArgs a{};
    a.q = static_cast<const half_t*>(q->data);
    a.k = static_cast<const half_t*>(k->data);
    a.v = static_cast<const half_t*>(v->data);
    a.bias = static_cast<const half_t*>(bias->data);
    a.kmask = static_cast<const uint8_t*>(kmask->data);
    a.out = static_cast<const half_t*>(out->data);
    a.dout = static_cast<const half_t*>(dout->data);
    a.lse = static_cast<const float*>(lse->data);
    a.dq = static_cast<half_t*>(dq->data);
    a.dk = static_cast<half_t*>(dk->data);
    a.dv = static_cast<half_t*>(dv->data);
    a.dbias = static_cast<float*>(dbias->data);
    char* ws = static_cast<char*>(workspace);
    a.qstat = reinterpret_cast<float*>(ws);
    a.biast = reinterpret_cast<float*>(ws + 2 * p.delta_bytes);
    a.partial = reinterpret_cast<float*>(ws + 2 * p.delta_bytes + p.biast_bytes);
    a.dkv = reinterpret_cast<float*>(ws + 2 * p.delta_bytes + p.biast_bytes + p.partial_bytes);
    a.bfrag = reinterpret_cast<half_t*>(ws + 2 * p.delta_bytes + p.biast_bytes + p.partial_bytes + p.dkv_bytes);
    a.N = (int)N; a.H = (int)H; a.Sq = (int)Sq; a.Sk = (int)Sk; a.D = (int)D;
    a.SqA = p.SqA;
    a.SqB = p.SqB;
    a.SkA = p.SkA;
    a.kblocks = p.kblocks;
    a.chunk = p.chunk;
    a.chunks = p.chunks;
    a.fn = fast_div(N);
    a.fkb = fast_div(p.kblocks);
    a.fch = fast_div(p.chunks);
    a.fwin = fast_div(p.windows);
    a.wtiles = p.wtiles;
    a.windows = p.windows;
    a.scale = scale;
    a.c1 = scale * kLog2e;
    a.kscale = fabsf(a.c1) >= 1e-30f;
    if (!a.kscale) a.c1 = 1.f;  // scale log2e S is below fp32 resolution against the bias
    a.c1s = a.c1 / kLog2e;
    a.rc1 = 1.f / a.c1;
    a.bias_vec = Sk % 8 == 0 && aligned16(a.bias);
    a.dbias_vec = Sk % 4 == 0 && aligned16(a.dbias);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (N * H * Sq == 0 || Sk == 0) {
        // no query or no key: every gradient is an empty sum (fp16 tensors have an even element
        // count since D is even)
        const int64_t nq = N * H * Sq * D, nk = N * H * Sk * D, nb = H * Sq * Sk;
        if (nq > 0) hipLaunchKernelGGL(fill_zero_f32, dim3(256), dim3(256), 0, s, static_cast<float*>(dq->data), nq / 2);
        if (nk > 0) {
            hipLaunchKernelGGL(fill_zero_f32, dim3(256), dim3(256), 0, s, static_cast<float*>(dk->data), nk / 2);
            hipLaunchKernelGGL(fill_zero_f32, dim3(256), dim3(256), 0, s, static_cast<float*>(dv->data), nk / 2);
        }
        if (nb > 0) hipLaunchKernelGGL(fill_zero_f32, dim3(256), dim3(256), 0, s, a.dbias, nb);
        return launch_status("attention_bwd");
    }
    if (p.DP == 32) return launch_bwd<32>(s, a, p, want_dbias);
    if (p.DP == 64) return launch_bwd<64>(s, a, p, want_dbias);
    return launch_bwd<96>(s, a, p, want_dbias);
}

extern "C" int clk_attention_bwd(clk_stream stream, int32_t device, const clk_buffer* q,
                                 const clk_buffer* k, const clk_buffer* v, const clk_buffer* bias,
                                 const clk_buffer* kmask, const clk_buffer* out,
                                 const clk_buffer* dout, const clk_buffer* lse,
                                 const clk_buffer* dq, const clk_buffer* dk, const clk_buffer* dv,
                                 const clk_buffer* dbias, float scale, int32_t want_dbias,
                                 void* workspace, size_t workspace_bytes) {
    return attention_bwd_impl(stream, device, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv,
                              dbias, scale, want_dbias, workspace, workspace_bytes, false);
}

extern "C" int clk_attention_bwd_noalloc(clk_stream stream, int32_t device, const clk_buffer* q,
                                         const clk_buffer* k, const clk_buffer* v,
                                         const clk_buffer* bias, const clk_buffer* kmask,
                                         const clk_buffer* out, const clk_buffer* dout,
                                         const clk_buffer* lse, const clk_buffer* dq,
                                         const clk_buffer* dk, const clk_buffer* dv,
                                         const clk_buffer* dbias, float scale,
                                         int32_t want_dbias) {
    return attention_bwd_impl(stream, device, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv,
                              dbias, scale, want_dbias, nullptr, 0, true);
}

extern "C" size_t clk_attention_bwd_noalloc_scratch_size(void) { return kNoAllocScratchBytes; }
