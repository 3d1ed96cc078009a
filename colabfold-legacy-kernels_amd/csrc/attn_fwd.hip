// Biased, masked, optionally gated flash-attention forward for gfx950 (CDNA4).
//
// Semantics follow the reference's VoltaMma / VoltaMmaPacked / VoltaMmaPackedTrim
// (cuda/volta_mma_attn.cu:115-465, 522-623): logits = scale q.k + bias[h,q,k] for a kept key,
// the masked logit -1e4 for a masked key (bias ignored), -inf past Sk; online softmax with the
// lazy max rule (the running max moves only when a tile raises it by more than 2^6 in the
// exp2 domain, decided per wave); P rounded to fp16 for the P.V product while l sums the fp32
// P; out = fp16(gate(O / max(l, 1e-30))); lse = m + log2 l in the log2 domain, -inf when l == 0.
//
// Layout on the chip. A workgroup is 4 waves and 128 queries of one (n, h): each wave owns 32
// queries as two 16-column MFMA blocks. Key tiles of 64 stream through LDS: K row-major (the A
// operand of S^T = K Q^T) and V transposed (the A operand of O^T = V^T P^T). Working in the
// transposed orientation keeps everything a lane touches on ONE query: the S^T accumulator of
// lane l holds keys 16 (l/16) + 4 kb + i of query l % 16, so the softmax statistics and the
// O rescale are per-lane scalars, P^T feeds the second MFMA as its B operand without leaving
// registers, and a lane's bias and mask are 16 contiguous elements of one row.
#include <type_traits>

#include "clk_common.h"

namespace clk {

struct FwdArgs {
    const half_t* q;
    const half_t* k;
    const half_t* v;
    const half_t* bias;
    const uint8_t* kmask;
    half_t* out;
    float* lse;
    const half_t* gate;       // same strides as q (the packed form's fourth slot), or null
    const half_t* gate_bias;  // [H, D]
    const int32_t* lims;      // [N + 1] (trim), or null
    int64_t qn, qh, qs, kn, kh, ks, on, oh, os;  // element strides of q/gate, k/v, out
    int N, H, Sq, Sk, D;
    float scale;
    int bias_vec;  // bias rows are whole 16-byte vectors (Sk % 8 == 0), one head's bias < 2^31 bytes
    int order;     // work-item order (ItemOrder)
    FastDiv fqt, fn, fh;  // division by the query tiles per (n, h), by N and by H (set at launch)
};

// Orders of the (n, h) work items, each item's query tiles consecutive. An XCD takes a contiguous
// run of items (xcd_item), so the order decides what its L2 holds at once:
// - kOrderHeads, head-major, for [N,H,S,D] tensors: a run covers few heads, so the bias rows it
//   reads stay in its L2;
// - kOrderHeadPairs, for packed rows with H even: head pairs outermost, then rows, then the two
//   heads of the pair. A row's K/V/gate values of heads 2j and 2j + 1 share 128-byte lines (at
//   D = 32), which the pair reads together, and a run's bias is two heads';
// - kOrderRows, for packed rows with H odd: the heads of one row together.
enum ItemOrder { kOrderRows = 0, kOrderHeads = 1, kOrderHeadPairs = 2 };

template <int DP>
struct FwdTile {
    static constexpr int kWaves = 4;
    static constexpr int kThreads = kWaves * kWave;
    static constexpr int kQB = 2;                     // 16-query MFMA blocks per wave
    static constexpr int kBQ = kWaves * kQB * 16;     // queries per workgroup
    static constexpr int kBK = 64;                    // keys per tile
    static constexpr int kKS = DP / 32;               // contraction steps of S^T
    static constexpr int kDB = DP / 16;               // 16-row blocks of O^T
    static constexpr int kKsLd = DP + 8;              // K and V row stride in LDS (halfs)
    static constexpr int kChunks = kBK * DP / 8;      // 16-byte chunks in a K (or V) tile
    static constexpr int kCPT = (kChunks + kThreads - 1) / kThreads;
    static constexpr int kLds = 2 * (2 * kBK * kKsLd) * 2;
};

struct H16 {
    half8 lo, hi;
};

__device__ __forceinline__ half8 zero8() {
    half8 z;
#pragma unroll
    for (int j = 0; j < 8; ++j) z[j] = (half_t)0.f;
    return z;
}

__device__ __forceinline__ half8 ld8(const half_t* p) { return *reinterpret_cast<const half8*>(p); }

// 16 consecutive halfs from p, elements at or past `valid` as 0
__device__ __forceinline__ H16 load_h16(const half_t* p, int valid, bool vec) {
    H16 r;
    if (vec && valid >= 16) {
        r.lo = ld8(p);
        r.hi = ld8(p + 8);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            r.lo[j] = j < valid ? p[j] : (half_t)0.f;
            r.hi[j] = j + 8 < valid ? p[j + 8] : (half_t)0.f;
        }
    }
    return r;
}

template <int DP, bool LSE, bool GATE, bool TRIM>
__global__ __launch_bounds__(FwdTile<DP>::kThreads, DP == 32 ? 3 : 1) void attn_fwd_kernel(FwdArgs a) {
    using T = FwdTile<DP>;
    // two key tiles in flight: one being read by the MFMAs, the next being written
    // (at DP = 32 four unpadded arrays instead, one per tensor and buffer: below)
    __shared__ __attribute__((aligned(16))) half_t Ks2[DP == 32 ? 1 : 2][T::kBK * T::kKsLd];
    __shared__ __attribute__((aligned(16))) half_t Vs2[DP == 32 ? 1 : 2][T::kBK * T::kKsLd];
    constexpr int kD32 = DP == 32 ? T::kBK * 32 : 8;
    __shared__ __attribute__((aligned(16))) half_t K32a[kD32], K32b[kD32], V32a[kD32], V32b[kD32];
    // where bias rows are whole 16-byte vectors: each wave's bias tiles (its 32 queries x 64 keys),
    // two buffers, filled by direct-to-LDS loads (below)
    __shared__ __attribute__((aligned(16))) half_t Bs[T::kWaves][2][4 * 520];

    const int item = xcd_item(blockIdx.x, gridDim.x);
    const int rest = fdiv(item, a.fqt), qt = item - rest * (int)a.fqt.d;
    int n, h;
    if (a.order == kOrderHeads) {
        h = fdiv(rest, a.fn);
        n = rest - h * a.N;
    } else if (a.order == kOrderHeadPairs) {
        const int pair = fdiv(rest >> 1, a.fn);
        n = (rest >> 1) - pair * a.N;
        h = 2 * pair + (rest & 1);
    } else {
        n = fdiv(rest, a.fh);
        h = rest - n * a.H;
    }
    const int q0 = qt * T::kBQ;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int r16 = lane & 15, g = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(wave);

    const int64_t qbase = n * a.qn + h * a.qh;
    const int64_t kbase = n * a.kn + h * a.kh;
    const int64_t obase = n * a.on + h * a.oh;

    int k_end = a.Sk;
    if constexpr (TRIM) {
        // a row with no live key, or a query tile past every row's live keys, is padding
        k_end = a.lims[n];
        if (k_end == 0 || q0 >= a.lims[a.N]) {
            const int cpr = a.D / 8;
            for (int i = tid; i < T::kBQ * cpr; i += T::kThreads) {
                const int r = i / cpr, c = (i - r * cpr) * 8, gq = q0 + r;
                if (gq < a.Sq) {
                    *reinterpret_cast<uint4*>(a.out + obase + gq * a.os + c) =
                        make_uint4(0u, 0u, 0u, 0u);
                }
            }
            return;
        }
    }

    // Q^T as the B operand of S^T: lane column q = q0w + 16 qb + r16, slots d = 32 ks + 8 g + j
    const int q0w = q0 + wave * (T::kQB * 16);
    // (loaded after the first key tile's loads are issued, so that their latencies overlap)
    half8 qop[T::kQB][T::kKS];
    const auto load_q = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int qb = 0; qb < T::kQB; ++qb) {
            const int gq = q0w + 16 * qb + r16;
#pragma unroll
            for (int ks = 0; ks < T::kKS; ++ks) {
                const int d0 = 32 * ks + 8 * g;
                qop[qb][ks] = (gq < a.Sq && d0 < a.D) ? ld8(a.q + qbase + gq * a.qs + d0) : zero8();
            }
        }
    };

    // running max m, its exp2-domain negative -m log2e and raise threshold m log2e + 6, and l
    float m_run[T::kQB], nm2[T::kQB], thr[T::kQB], l_run[T::kQB];
    float4v acc[T::kDB][T::kQB];
#pragma unroll
    for (int qb = 0; qb < T::kQB; ++qb) {
        m_run[qb] = -INFINITY;
        nm2[qb] = 0.f;
        thr[qb] = -INFINITY;
        l_run[qb] = 0.f;
#pragma unroll
        for (int db = 0; db < T::kDB; ++db) acc[db][qb] = float4v{0.f, 0.f, 0.f, 0.f};
    }

    const float scale = a.scale;

    // K/V chunks of the next key tile, held in registers one tile ahead of their LDS store. A
    // chunk's row and column are fixed per lane; the loads are buffer loads whose range is the
    // tile's rows below Sk, so a row past Sk and a column past D read zeros. Lane l of every wave
    // also loads the mask byte of key k0 + l (zero past Sk): a wave ballot of those bytes is the
    // tile's keep bits, uniform across the workgroup. A masked key's K row is staged as zeros,
    // so its score is exactly 0 and its bias register (which then holds the masked logit) is its
    // logit.
    uint32_t kvoff[T::kCPT];
    int krow[T::kCPT], kdst[T::kCPT], vdst[T::kCPT];
#pragma unroll
    for (int i = 0; i < T::kCPT; ++i) {
        const int c = tid + i * T::kThreads;  // kChunks = kCPT kThreads
        const int row = c / (DP / 8), col = (c - row * (DP / 8)) * 8;
        kvoff[i] = col < a.D ? (uint32_t)((row * a.ks + col) * 2) : 0x80000000u;
        krow[i] = row;
        // K fragment-major: the A operand of key block kb, step ks is 64 consecutive 16-byte chunks
        // (lane r + 16 g: key 16 (r/4) + 4 kb + r%4, d 32 ks + 8 g ..), so each read is one
        // conflict-free 1 KB sweep
        const int kb = (row >> 2) & 3, r16 = 4 * (row >> 4) + (row & 3);
        kdst[i] = ((kb * T::kKS + (col >> 5)) * kWave + r16 + 16 * ((col >> 3) & 3)) * 8;
        vdst[i] = row * T::kKsLd + col;
    }
    const char* const kb_base = reinterpret_cast<const char*>(a.k + kbase);
    const char* const vb_base = reinterpret_cast<const char*>(a.v + kbase);
    const char* const mrow = reinterpret_cast<const char*>(a.kmask + (int64_t)n * a.Sk);
    half8 kreg[T::kCPT], vreg[T::kCPT];
    uint32_t mbyte = 0u;
    const auto fetch = [&](int k0) {
        const int rows = min(a.Sk - k0, T::kBK);
        const int64_t kofs = (int64_t)k0 * a.ks * 2;
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kb_base + kofs), 0,
                                                          rows * (int)a.ks * 2, 0x00020000);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vb_base + kofs), 0,
                                                          rows * (int)a.ks * 2, 0x00020000);
#pragma unroll
        for (int i = 0; i < T::kCPT; ++i) {
            kreg[i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rk, kvoff[i], 0, 0));
            vreg[i] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rv, kvoff[i], 0, 0));
        }
        const auto rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(mrow + k0), 0, rows, 0x00020000);
        mbyte = __builtin_amdgcn_raw_buffer_load_b8(rm, (uint32_t)lane, 0, 0);
    };
    // Dead keys of a tile whose bias came through LDS, when they are few: each takes its logit in
    // the wave's own bias tile before the tile's reads, one LDS store per key from the wave's
    // first 32 lanes (one query row each) in a scalar loop over the keys (the keep ballot is
    // uniform): the masked logit inside Sk, -inf past it. Tiles with more dead keys fix the bias
    // registers instead (fix_bias, a fixed cost per tile). At DP = 32 the stores go with the
    // tile's K zeroing, in stage's wait for the tile's loads (a branch that only tiles with a
    // dead key take), so a tile loop without dead keys carries none of this code; other widths
    // store at the start of the tile, after its wait for the bias loads.
    typedef __attribute__((address_space(3))) char lds_char;
    const auto kill_bias_lds = [&](int bb, int k0, uint64_t keep64) {
        if (lane >= 32) return;
        const int kvalid = a.Sk - k0;
        const uint64_t inside = kvalid >= 64 ? ~0ull : (1ull << kvalid) - 1ull;
        // (the lane's row base and swizzle, formed here rather than kept live through the kernel)
        lds_char* const row = (lds_char*)(&Bs[wv][bb][0]) + 1040 * ((lane & 31) >> 3) + 128 * (lane & 7);
        const uint32_t kill_x = 32u * (uint32_t)((lane & 7) >> 1);
        const auto put = [&](uint64_t keys, half_t v) {
            while (keys) {
                const uint32_t k = (uint32_t)__builtin_ctzll(keys);
                keys &= keys - 1ull;
                *reinterpret_cast<__attribute__((address_space(3))) half_t*>(row + ((2u * k) ^ kill_x)) = v;
            }
        };
        put(~keep64 & inside, (half_t)kMaskedLogit);
        put(~keep64 & ~inside, (half_t)(-INFINITY));
    };
    constexpr int kKillMax = 8;  // most dead keys per tile that go through LDS stores
    const auto stage = [&](auto vec, int buf, int k0, uint64_t keep) {
        if constexpr (DP == 32) {
            // the tile came by direct-to-LDS loads (below): once they have landed, each wave
            // zeroes the K rows of the masked keys in its own fragment block, and where its bias
            // came through LDS too, writes a few dead keys' logits into its bias tile
            if (keep != ~0ull) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                const int key = 16 * ((lane & 15) >> 2) + 4 * wv + (lane & 3);
                if (!((keep >> key) & 1u))
                    *reinterpret_cast<half8*>((buf ? K32b : K32a) + 512 * wv + 8 * lane) = zero8();
                if constexpr (decltype(vec)::value) {
                    if (__builtin_popcountll(~keep) <= kKillMax) kill_bias_lds(buf, k0, keep);
                }
            }
        } else {
            half_t* Ks = Ks2[buf];
            half_t* Vs = Vs2[buf];
#pragma unroll
            for (int i = 0; i < T::kCPT; ++i) {
                *reinterpret_cast<half8*>(&Ks[kdst[i]]) = (keep >> krow[i]) & 1u ? kreg[i] : zero8();
                *reinterpret_cast<half8*>(&Vs[vdst[i]]) = vreg[i];
            }
        }
    };
    // At DP = 32 the K and V tiles go from memory straight into LDS by direct-to-LDS loads
    // (buffer_load ... lds), one 1 KB load of each per wave, issued with the next tile's other
    // loads and complete at the tile's closing barrier: no staging registers and no LDS stores.
    // Wave w loads K's fragment block w (slot l: key 16 (l % 16 / 4) + 4 w + l % 4, d 8 (l / 16)
    // .. +7, the layout above) and V rows 16 w .. +15 unpadded (slot l: row 16 w + l / 4, d
    // 8 (l % 4) ..). Masked keys' K rows are zeroed in LDS after the loads land (stage).
    uint32_t kdma = 0u, vdma = 0u;
    if constexpr (DP == 32) {
        const int kr = 16 * ((lane & 15) >> 2) + 4 * wave + (lane & 3), kc = 8 * (lane >> 4);
        const int vr = 16 * wave + (lane >> 2), vc = 8 * (lane & 3);
        kdma = kc < a.D ? (uint32_t)((kr * a.ks + kc) * 2) : 0x80000000u;
        vdma = vc < a.D ? (uint32_t)((vr * a.ks + vc) * 2) : 0x80000000u;
    }
    const auto dma_kv = [&](int k0, int buf) {
        const int rows = min(a.Sk - k0, T::kBK);
        const int64_t kofs = (int64_t)k0 * a.ks * 2;
        // (a wave-uniform range, kept in a scalar register: the loads need scalar descriptors)
        const int range = __builtin_amdgcn_readfirstlane(rows * (int)a.ks * 2);
        const auto rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(kb_base + kofs), 0, range, 0x00020000);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vb_base + kofs), 0, range, 0x00020000);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rk, (__attribute__((address_space(3))) void*)((buf ? K32b : K32a) + 512 * wv), 16, kdma, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rv, (__attribute__((address_space(3))) void*)((buf ? V32b : V32a) + 512 * wv), 16, vdma, 0, 0, 0);
        const auto rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(mrow + k0), 0, rows, 0x00020000);
        mbyte = __builtin_amdgcn_raw_buffer_load_b8(rm, (uint32_t)lane, 0, 0);
    };
    // the next tile's K, V and mask byte into buffer buf
    const auto fetch_kv = [&](int k0, int buf) {
        if constexpr (DP == 32) {
            dma_kv(k0, buf);
        } else {
            fetch(k0);
        }
    };
    // Gated at DP = 32: the last key tile loads, in place of a next tile, the wave's gate rows into
    // the idle buffer's regions of this wave (its K fragment block: query block 0, its V rows:
    // block 1), so the epilogue's gate reads are LDS reads whose memory latency the last tile
    // covered. Slot l of block qb is query q0w + 16 qb + R (R = l / 4), 16-byte chunk
    // c = (l % 4) ^ (R / 4) % 4 of the row, at byte 16 l; rows past Sq and chunks past D read zeros.
    bool gate_lds = false;
    const auto dma_gate = [&](int buf) {
        const int R = lane >> 2, c = (lane & 3) ^ ((R >> 2) & 3);
        const int rows = max(a.Sq - q0w, 0);
        const int range = __builtin_amdgcn_readfirstlane(min(rows, T::kQB * 16) * (int)a.qs * 2);
        const auto rg = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.gate + qbase + (int64_t)q0w * a.qs),
                                                          0, range, 0x00020000);
#pragma unroll
        for (int qb = 0; qb < T::kQB; ++qb) {
            const uint32_t off = 8 * c < a.D ? (uint32_t)(((16 * qb + R) * a.qs + 8 * c) * 2) : 0x80000000u;
            half_t* dst = (qb == 0 ? (buf ? K32b : K32a) : (buf ? V32b : V32a)) + 512 * wv;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (__attribute__((address_space(3))) void*)dst, 16, off, 0, 0, 0);
        }
        // and the head's gate bias (D halfs) into the wave's idle bias buffer of that parity
        const auto rgb = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(a.gate_bias + (int64_t)h * a.D), 0,
                                                           a.D * 2, 0x00020000);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rgb, (__attribute__((address_space(3))) void*)&Bs[wv][buf][0], 16,
                                                 16u * (uint32_t)lane, 0, 0, 0);
        gate_lds = true;
    };
    int gate_buf = 0;

    // bias of this lane's 16 keys k0 + 16 g .. +15 for its queries, in a register set per tile
    // parity: loaded one key tile ahead where rows are not whole 16-byte vectors, else read from
    // LDS at the start of the tile (below); when the tile comes up, a masked key's bias becomes
    // the masked logit -1e4 and a key past Sk's -inf
    // (the register path's row pointers: brow, set where that path starts)
    const half_t* brow[T::kQB];
    const auto set_brow = [&]() {
#pragma unroll
        for (int qb = 0; qb < T::kQB; ++qb) {
            const int gq = q0w + 16 * qb + r16;
            const int gqc = gq < a.Sq ? gq : a.Sq - 1;
            brow[qb] = a.bias + (int64_t)h * a.Sq * a.Sk + (int64_t)gqc * a.Sk + 16 * g;
        }
    };
    // Where bias rows are whole 16-byte vectors (and a head's bias spans under 2^31 bytes) the
    // bias goes through LDS: a lane's 16 keys of one query row are 32 bytes of a different row
    // for each of 16 lanes, so register loads of them touch 16 cache lines per instruction, which
    // measured a sixth of the kernel's time. Instead the wave loads its 32 x 64 bias tile with
    // four direct-to-LDS loads (buffer_load ... lds) from a buffer whose range is the head's bias
    // block, each a contiguous sweep of 8 rows x 128 bytes: lane 8 r + j of load m reads row 8 m + r,
    // 16-byte segment j ^ 2 (r / 2), and lands at byte 1040 m + 16 (8 r + j) of the wave's buffer,
    // so key k of row 8 m + r sits at byte 1040 m + 128 r + (2 k ^ 32 (r / 2)). The swizzle and the
    // 16-byte skew between loads put the 16 rows of each 16-lane read on distinct LDS banks. Rows past Sq lie past the buffer's range and read zeros (their
    // results are never stored); keys past Sk read the next row's values or zeros and become -inf
    // when their tile comes up.
    const half_t* const bias_head = a.bias + (int64_t)h * a.Sq * a.Sk;
    uint32_t bdma[4];
    {
        const int r = lane >> 3, seg = (lane & 7) ^ (2 * (r >> 1));
        bdma[0] = (uint32_t)(q0w + r) * (uint32_t)a.Sk * 2u + 16u * (uint32_t)seg;
#pragma unroll
        for (int m = 1; m < 4; ++m) bdma[m] = bdma[0] + (uint32_t)m * 16u * (uint32_t)a.Sk;
    }
    const auto dma_bias = [&](int k0, int bb) {
        const auto rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(bias_head + k0), 0,
                                                          (a.Sq * a.Sk - k0) * 2, 0x00020000);
#pragma unroll
        for (int m = 0; m < 4; ++m)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (__attribute__((address_space(3))) void*)&Bs[wv][bb][520 * m], 16, bdma[m], 0, 0, 0);
    };
    // this lane's 16 keys of query row 16 qb + r16 from the wave's buffer bb: segments 2 g and
    // 2 g + 1, adjacent in LDS
    const auto read_bias = [&](int bb, H16 (&b)[T::kQB]) {
#pragma unroll
        for (int qb = 0; qb < T::kQB; ++qb) {
            const int m = 2 * qb + (r16 >> 3), r = r16 & 7;
            const half_t* p = &Bs[wv][bb][520 * m + 8 * (8 * r + ((2 * g) ^ (2 * (r >> 1))))];
            b[qb].lo = ld8(p);
            b[qb].hi = ld8(p + 8);
        }
    };
    const auto fetch_bias = [&](int k0, H16 (&b)[T::kQB]) {
        if (a.bias_vec && k0 + T::kBK <= a.Sk) {
#pragma unroll
            for (int qb = 0; qb < T::kQB; ++qb) {
                b[qb].lo = ld8(brow[qb] + k0);
                b[qb].hi = ld8(brow[qb] + k0 + 8);
            }
        } else {
#pragma unroll
            for (int qb = 0; qb < T::kQB; ++qb) b[qb] = load_h16(brow[qb] + k0, a.Sk - (k0 + 16 * g), a.bias_vec);
        }
    };
    const auto fix_bias = [&](int k0, H16 (&b)[T::kQB], uint64_t keep64) {
        if (k0 + T::kBK <= a.Sk) {
            // every key of the tile inside Sk (a uniform test): only the masked logit fills in
            const uint32_t keep = (uint32_t)(keep64 >> (16 * g)) & 0xffffu;
            if (keep != 0xffffu) {
#pragma unroll
                for (int qb = 0; qb < T::kQB; ++qb)
                    fill_bias16(b[qb].lo, b[qb].hi, keep, 0xffffu, (half_t)kMaskedLogit, (half_t)kMaskedLogit);
            }
        } else {
            const int kvalid = a.Sk - (k0 + 16 * g);
            const uint32_t inside = kvalid >= 16 ? 0xffffu : kvalid <= 0 ? 0u : (1u << kvalid) - 1u;
            const uint32_t keep = (uint32_t)(keep64 >> (16 * g)) & inside;
            if (keep != 0xffffu) {
#pragma unroll
                for (int qb = 0; qb < T::kQB; ++qb)
                    fill_bias16(b[qb].lo, b[qb].hi, keep, inside, (half_t)kMaskedLogit, (half_t)(-INFINITY));
            }
        }
    };

    // One key tile: prefetch the next, then S^T, the online softmax and O^T += V^T P^T. On the
    // vector path every prefetch load is issued unconditionally (the last tile loads and stages
    // itself again into the idle buffer), so the tile is straight-line code and each wait
    // covers only the loads it needs.
    uint64_t keep_cur = 0u;
    const int k_last = (k_end - 1) / T::kBK * T::kBK;
    const auto tile = [&](auto vec, auto first, int k0, int buf, H16 (&bias16)[T::kQB],
                          H16 (&bias_next)[T::kQB]) __attribute__((always_inline)) {
        const half_t* Ks = DP == 32 ? (buf ? K32b : K32a) : Ks2[buf & (DP == 32 ? 0 : 1)];
        const half_t* Vs = DP == 32 ? (buf ? V32b : V32a) : Vs2[buf & (DP == 32 ? 0 : 1)];
        bool more = true;
        bool reg_fix = keep_cur != ~0ull;
        int k_next = k0 + T::kBK;
        if constexpr (decltype(vec)::value) {
            // this tile's bias loads, issued a tile ago, are the only loads in flight: wait for
            // them (the compiler does not order LDS reads after direct-to-LDS loads by itself)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            // (keys past Sk read as dead: their mask bytes load as zero)
            reg_fix = keep_cur != ~0ull && __builtin_popcountll(~keep_cur) > kKillMax;
            if constexpr (DP != 32) {
                if (keep_cur != ~0ull && !reg_fix) kill_bias_lds(buf, k0, keep_cur);
            }
            read_bias(buf, bias16);
            k_next = min(k0 + T::kBK, k_last);
            if (GATE && DP == 32 && k0 == k_last) {
                dma_gate(buf ^ 1);
                gate_buf = buf ^ 1;
                more = false;
            } else {
                fetch_kv(k_next, buf ^ 1);
                dma_bias(k_next, buf ^ 1);
            }
        } else {
            more = k0 + T::kBK < k_end;
            if (more) {
                fetch_kv(k0 + T::kBK, buf ^ 1);
                fetch_bias(k0 + T::kBK, bias_next);
            } else if constexpr (GATE && DP == 32) {
                dma_gate(buf ^ 1);
                gate_buf = buf ^ 1;
            }
        }
        // every key of the tile kept and inside Sk: the bias stands as loaded (through LDS a few
        // dead keys' logits are in place already)
        if (reg_fix) fix_bias(k0, bias16, keep_cur);

        // S^T = K Q^T: A row r of key block kb is key 16 (r/4) + 4 kb + r%4, fragment-major;
        // then the natural-domain logits t = scale s + bias: a masked key's s is 0 (its K row
        // staged as zeros) and its bias the masked logit, a key past Sk has bias -inf
        float4v s[4][T::kQB];
        const auto logits = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int qb = 0; qb < T::kQB; ++qb) s[kb][qb] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < T::kKS; ++ks) {
                    const half8 kop = ld8(&Ks[((kb * T::kKS + ks) * kWave + lane) * 8]);
#pragma unroll
                    for (int qb = 0; qb < T::kQB; ++qb) s[kb][qb] = mfma16x16x32(kop, qop[qb][ks], s[kb][qb]);
                }
            }
#pragma unroll
            for (int qb = 0; qb < T::kQB; ++qb)
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int kk = 4 * kb + i;
                        const half_t b = kk < 8 ? bias16[qb].lo[kk] : bias16[qb].hi[kk - 8];
                        s[kb][qb][i] = fmaf(s[kb][qb][i], scale, (float)b);
                    }
        };
        logits();

        // lazy max: move only when some query of the wave gains more than 6 in log2 units. A
        // query's tile max is the largest of its four lanes' maxima, so the per-lane test decides
        // the same; the cross-lane maximum is only needed on a tile that raises. Returns whether
        // the wave moved (always on the first tile, where thr is -inf).
        const auto lazy_max = [&]() __attribute__((always_inline)) -> bool {
            float m_tile[T::kQB];
            bool up = false;
#pragma unroll
            for (int qb = 0; qb < T::kQB; ++qb) {
                float mx = s[0][qb][0];
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[kb][qb][i]);
                m_tile[qb] = mx;
                up |= m_tile[qb] * kLog2e > thr[qb];
            }
            if (!__any(up)) return false;
            // the running max moves: rescale l and O by 2^(m - m_new)
#pragma unroll
            for (int qb = 0; qb < T::kQB; ++qb) {
                const float m_new = fmaxf(m_run[qb], wave_xor_max4(m_tile[qb]));
                // (before the first move l and O are still zero: nothing to rescale)
                if (m_run[qb] > -INFINITY) {
                    const float alpha = exp2_fast((m_run[qb] - m_new) * kLog2e);
                    l_run[qb] *= alpha;
#pragma unroll
                    for (int db = 0; db < T::kDB; ++db) acc[db][qb] *= alpha;
                }
                m_run[qb] = m_new;
                nm2[qb] = -m_new * kLog2e;
                thr[qb] = m_new * kLog2e + 6.f;
            }
            return true;
        };

        // p = 2^(t log2e - m log2e), packed to fp16 for the P.V product, and the tile's fp32 sum
        // of p per query (of this lane's 16 keys)
        half8 pb[2][T::kQB];
        float lt[T::kQB];
        const auto probs = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (int qb = 0; qb < T::kQB; ++qb) {
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float p = exp2_fast(fmaf(s[kb][qb][i], kLog2e, nm2[qb]));
                        lt[qb] = kb == 0 && i == 0 ? p : lt[qb] + p;
                        pb[kb >> 1][qb][4 * (kb & 1) + i] = (half_t)p;
                    }
                }
            }
        };
        if constexpr (decltype(first)::value) {
            lazy_max();
            probs();
        } else {
            // A logit above the running max by more than 6 has p > 2^6; p >= 0, so a lane whose
            // 16 p of a query sum to at most 64 holds none for that query. Only a wave where some
            // lane's sum exceeds 64 takes the exact test, on the logits formed again (bias
            // included) rather than kept live through the tile, and p again if the max moved.
            probs();
            bool hot = false;
#pragma unroll
            for (int qb = 0; qb < T::kQB; ++qb) hot |= !(lt[qb] <= 64.f);
            if (__any(hot)) {
                if constexpr (decltype(vec)::value) {
                    read_bias(buf, bias16);
                    if (reg_fix) fix_bias(k0, bias16, keep_cur);
                }
                logits();
                if (lazy_max()) probs();
            }
        }
#pragma unroll
        for (int qb = 0; qb < T::kQB; ++qb) l_run[qb] += lt[qb];

        // O^T += V^T P^T: A row r of d block db is d = (DP/4)(r/4) + 4 db + r%4; slot 8 g + j of
        // contraction step kt is key 16 g + 8 kt + j, which is where P^T already sits. V^T is
        // read transposed from the row-major V tile.
        const auto vrow = [&](int r) { return Vs + r * (DP == 32 ? 32 : T::kKsLd); };
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int db = 0; db < T::kDB; ++db) {
                const half8 vop = lds_operand_tr(vrow, 2 * g + kt, r16, 4 * db, DP / 4);
#pragma unroll
                for (int qb = 0; qb < T::kQB; ++qb) acc[db][qb] = mfma16x16x32(vop, pb[kt][qb], acc[db][qb]);
            }
        }
        // the other buffer was last read a tile ago, before the barrier that ended that tile
        if (more) {
            keep_cur = __ballot(mbyte != 0u);
            stage(vec, buf ^ 1, k_next, keep_cur);
        }
        // at DP = 32 the next tile's K and V, loaded straight into LDS at the start of this tile,
        // have landed before the barrier after which every wave reads them (the compiler also
        // waits for all loads before a barrier; the order does not rest on it)
        if constexpr (DP == 32) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };

    // A row whose first key tile holds no live key may hold none at all: then every key inside Sk
    // has the masked logit, the softmax is uniform, and the tile loop would produce out = the mean
    // of the row's V rows and lse2 = -1e4 log2 e + log2 Sk. Such a workgroup (rows of padded
    // residues) sums V instead: wave w takes rows r16 + 16 (w + 4 i), lane group g its d's, and
    // the waves' sums meet in their own LDS bias buffers; the epilogue then divides by l = Sk.
    const auto dead_row = [&]() -> bool {
        bool live = false;
        for (int k = T::kBK + lane; k < a.Sk; k += kWave) live |= mrow[k] != 0;
        return !__any(live);
    };
    const auto dead_row_sums = [&]() {
        float sv[DP / 4];
#pragma unroll
        for (int e = 0; e < DP / 4; ++e) sv[e] = 0.f;
        const int range = __builtin_amdgcn_readfirstlane(a.Sk * (int)a.ks * 2);
        const auto rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(vb_base), 0, range, 0x00020000);
        for (int k = r16 + 16 * wv; k < a.Sk; k += 16 * T::kWaves) {
#pragma unroll
            for (int c = 0; c < DP / 32; ++c) {
                const int d0 = (DP / 4) * g + 8 * c;
                const uint32_t off = d0 < a.D ? (uint32_t)((k * a.ks + d0) * 2) : 0x80000000u;
                const half8 v = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
#pragma unroll
                for (int j = 0; j < 8; ++j) sv[8 * c + j] += (float)v[j];
            }
        }
#pragma unroll
        for (int e = 0; e < DP / 4; ++e)
#pragma unroll
            for (int m = 1; m < 16; m <<= 1) sv[e] += __shfl_xor(sv[e], m);
        // the first tile's loads into this wave's LDS have landed before its buffer takes the sums
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        if (r16 == 0) {
#pragma unroll
            for (int e = 0; e < DP / 4; ++e) reinterpret_cast<float*>(&Bs[wv][0][0])[(DP / 4) * g + e] = sv[e];
        }
        __syncthreads();
        float tot[DP / 4];
#pragma unroll
        for (int e = 0; e < DP / 4; ++e) {
            tot[e] = 0.f;
#pragma unroll
            for (int w = 0; w < T::kWaves; ++w) tot[e] += reinterpret_cast<const float*>(&Bs[w][0][0])[(DP / 4) * g + e];
        }
#pragma unroll
        for (int qb = 0; qb < T::kQB; ++qb) {
#pragma unroll
            for (int db = 0; db < T::kDB; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[db][qb][i] = tot[4 * db + i];
            l_run[qb] = g == 0 ? (float)a.Sk : 0.f;
            m_run[qb] = kMaskedLogit;
        }
    };

    H16 biasA[T::kQB], biasB[T::kQB];
    const auto run = [&](auto vec) __attribute__((always_inline)) {
        fetch_kv(0, 0);
        if constexpr (decltype(vec)::value) {
            dma_bias(0, 0);
        } else {
            set_brow();
            fetch_bias(0, biasA);
        }
        load_q();
        keep_cur = __ballot(mbyte != 0u);
        if constexpr (!TRIM) {
            if (keep_cur == 0ull && dead_row()) {
                dead_row_sums();
                return;
            }
        }
        stage(vec, 0, 0, keep_cur);
        __syncthreads();
        tile(vec, std::true_type{}, 0, 0, biasA, biasB);
        for (int k0 = T::kBK; k0 < k_end; k0 += 2 * T::kBK) {
            tile(vec, std::false_type{}, k0, 1, biasB, biasA);
            if (k0 + T::kBK < k_end) tile(vec, std::false_type{}, k0 + T::kBK, 0, biasA, biasB);
        }
        // the last tile's bias loads (of itself, unused) land before the workgroup's LDS is freed
        if constexpr (decltype(vec)::value) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
    if (k_end > 0) {
        if (a.bias_vec) {
            run(std::true_type{});
        } else {
            run(std::false_type{});
        }
    }

    // epilogue: lane g holds d = (DP/4) g .. +DP/4 of query q0w + 16 qb + r16. Gated, out =
    // acc / (l (1 + 2^(-(gate + gate_bias) log2 e))): one reciprocal per element covers both the
    // softmax normalisation and the sigmoid, and -gate_bias log2 e is formed once per lane.
    float ngb[DP / 32][8];
    if constexpr (GATE) {
#pragma unroll
        for (int c = 0; c < DP / 32; ++c) {
            // (a chunk past D, never stored, reads the last chunk: the loads need no guard)
            const int d0 = min((DP / 4) * g + 8 * c, a.D - 8);
            const half8 gb = DP == 32 && gate_lds ? ld8(&Bs[wv][gate_buf][d0]) : ld8(a.gate_bias + h * a.D + d0);
#pragma unroll
            for (int j = 0; j < 8; ++j) ngb[c][j] = -kLog2e * (float)gb[j];
        }
    }
#pragma unroll
    for (int qb = 0; qb < T::kQB; ++qb) {
        const int gq = q0w + 16 * qb + r16;
        const float l = wave_xor_sum4(l_run[qb]);
        if (gq >= a.Sq) continue;
        if constexpr (LSE) {
            if (g == 0) {
                a.lse[((int64_t)n * a.H + h) * a.Sq + gq] =
                    l > 0.f ? m_run[qb] * kLog2e + log2f(l) : -INFINITY;
            }
        }
        const float lc = fmaxf(l, 1e-30f);
        const float inv = GATE ? 0.f : __builtin_amdgcn_rcpf(lc);
#pragma unroll
        for (int c = 0; c < DP / 32; ++c) {
            const int d0 = (DP / 4) * g + 8 * c;
            if (d0 >= a.D) continue;
            half8 o;
            half8 gt;
            if constexpr (GATE) {
                if (DP == 32 && gate_lds) {
                    // (the final wait for loads at the end of the tile loop covers the gate rows)
                    const half_t* gl = (qb == 0 ? (gate_buf ? K32b : K32a) : (gate_buf ? V32b : V32a)) + 512 * wv;
                    gt = ld8(gl + 32 * r16 + 8 * (g ^ ((r16 >> 2) & 3)));
                } else {
                    gt = ld8(a.gate + qbase + gq * a.qs + d0);
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int db = 2 * c + j / 4, i = j & 3;
                float val;
                if constexpr (GATE) {
                    const float e = exp2_fast(fmaf((float)gt[j], -kLog2e, ngb[c][j]));
                    val = acc[db][qb][i] * __builtin_amdgcn_rcpf(fmaf(lc, e, lc));
                } else {
                    val = acc[db][qb][i] * inv;
                }
                o[j] = (half_t)val;
            }
            *reinterpret_cast<half8*>(a.out + obase + gq * a.os + d0) = o;
        }
    }
}

template <int DP, bool LSE, bool GATE, bool TRIM>
static int launch_fwd(hipStream_t stream, int device, const FwdArgs& a) {
    using T = FwdTile<DP>;
    const int max_smem = shared_limit(device);
    if (max_smem > 0 && T::kLds > max_smem) {
        return invalid("attention: needs " + std::to_string(T::kLds / 1024) +
                       " KB shared, device allows " + std::to_string(max_smem / 1024) + " KB");
    }
    const int64_t qt = (a.Sq + T::kBQ - 1) / T::kBQ;
    const int64_t grid = qt * a.H * a.N;
    if (grid == 0) return ok();
    if (grid > INT32_MAX) return invalid("attention: too many work items");
    FwdArgs b = a;
    b.fqt = fast_div(qt);
    b.fn = fast_div(a.N);
    b.fh = fast_div(a.H);
    stage_mark(stream, 0);
    hipLaunchKernelGGL((attn_fwd_kernel<DP, LSE, GATE, TRIM>), dim3((unsigned)grid),
                       dim3(T::kThreads), 0, stream, b);
    stage_mark(stream, 1);
    return launch_status("attention");
}

// The (D, block_q, block_k) entries the reference dispatches (volta_mma_attn.cu:508-517). The
// gfx950 kernel picks its own tiling per D; the table keeps the FFI contract, so a call the
// reference rejects is rejected here too.
static bool fwd_config_ok(int64_t d, int64_t bq, int64_t bk) {
    static const int64_t table[][3] = {
        {8, 64, 64},  {8, 64, 32},  {8, 32, 32},  {8, 128, 64}, {8, 32, 64},  {32, 64, 64},
        {32, 64, 32}, {32, 32, 64}, {32, 32, 32}, {32, 128, 64}, {32, 16, 64}, {16, 64, 64},
        {16, 32, 32}, {16, 64, 32}, {64, 64, 64}, {64, 32, 32}, {24, 64, 32}, {24, 32, 32},
        {48, 64, 32}, {48, 32, 32}, {96, 64, 32}, {96, 32, 32}};
    for (const auto& e : table)
        if (e[0] == d && e[1] == bq && e[2] == bk) return true;
    return false;
}

template <bool LSE, bool GATE, bool TRIM>
static int dispatch_fwd(hipStream_t stream, int device, const FwdArgs& a) {
    if (a.D <= 32) return launch_fwd<32, LSE, GATE, TRIM>(stream, device, a);
    if (a.D <= 64) return launch_fwd<64, LSE, GATE, TRIM>(stream, device, a);
    return launch_fwd<96, LSE, GATE, TRIM>(stream, device, a);
}

static FwdArgs contiguous_args(int N, int H, int Sq, int Sk, int D) {
    FwdArgs a{};
    a.qn = (int64_t)H * Sq * D;
    a.qh = (int64_t)Sq * D;
    a.qs = D;
    a.kn = (int64_t)H * Sk * D;
    a.kh = (int64_t)Sk * D;
    a.ks = D;
    a.on = a.qn;
    a.oh = a.qh;
    a.os = D;
    a.N = N;
    a.H = H;
    a.Sq = Sq;
    a.Sk = Sk;
    a.D = D;
    a.order = kOrderHeads;
    return a;
}

}  // namespace clk

using namespace clk;

extern "C" int clk_attention_fwd(clk_stream stream, int32_t device, const clk_buffer* q,
                                 const clk_buffer* k, const clk_buffer* v, const clk_buffer* bias,
                                 const clk_buffer* kmask, const clk_buffer* out,
                                 const clk_buffer* lse, float scale, int64_t block_q,
                                 int64_t block_k, int32_t want_lse) {
    const clk_buffer* bufs[] = {q, k, v, bias, kmask, out, lse};
    const int types[] = {CLK_F16, CLK_F16, CLK_F16, CLK_F16, CLK_U8, CLK_F16, CLK_F32};
    if (int st = check_types("attention", bufs, types, 7)) return st;
    if (q->rank != 4) return invalid("q must be [N,H,S,D]");
    const int64_t N = q->dims[0], H = q->dims[1], Sq = q->dims[2], D = q->dims[3];
    if (k->rank != 4 || k->dims[0] != N || k->dims[1] != H || k->dims[3] != D || !same_shape(v, k)) {
        return invalid("attention: k and v must be [N,H,Sk,D] like q");
    }
    const int64_t Sk = k->dims[2];
    if (!same_shape(out, q)) return invalid("attention: out must match q");
    if (elements(bias) != H * Sq * Sk || elements(kmask) != N * Sk) {
        return invalid("attention: bias must be [H,Sq,Sk] and kmask [N,Sk]");
    }
    if (want_lse && elements(lse) != N * H * Sq) return invalid("attention: lse must be [N,H,Sq]");
    if (!fwd_config_ok(D, block_q, block_k)) return invalid("volta_mma: unsupported (D, bq, bk)");
    if (!aligned16(q->data) || !aligned16(k->data) || !aligned16(v->data) || !aligned16(out->data)) {
        return invalid("attention: q, k, v and out must be 16-byte aligned");
    }
    if (N * H * Sq == 0) return ok();
    FwdArgs a = contiguous_args((int)N, (int)H, (int)Sq, (int)Sk, (int)D);
    a.q = static_cast<const half_t*>(q->data);
    a.k = static_cast<const half_t*>(k->data);
    a.v = static_cast<const half_t*>(v->data);
    a.bias = static_cast<const half_t*>(bias->data);
    a.kmask = static_cast<const uint8_t*>(kmask->data);
    a.out = static_cast<half_t*>(out->data);
    a.lse = want_lse ? static_cast<float*>(lse->data) : nullptr;
    a.scale = scale;
    a.bias_vec = Sk % 8 == 0 && aligned16(a.bias) && (int64_t)Sq * Sk * 2 < ((int64_t)1 << 31);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    return want_lse ? dispatch_fwd<true, false, false>(s, device, a)
                    : dispatch_fwd<false, false, false>(s, device, a);
}

static int packed_common(clk_stream stream, int32_t device, const clk_buffer* p,
                         const clk_buffer* bias, const clk_buffer* kmask,
                         const clk_buffer* gate_bias, const clk_buffer* lims,
                         const clk_buffer* out, float scale, int64_t block_q, int64_t block_k,
                         int32_t column) {
    const char* what = lims ? "attention_packed_trim" : "attention_packed";
    const clk_buffer* bufs[] = {p, bias, kmask, gate_bias, out, lims};
    const int types[] = {CLK_F16, CLK_F16, CLK_U8, CLK_F16, CLK_F16, CLK_S32};
    if (int st = check_types(what, bufs, types, lims ? 6 : 5)) return st;
    if (p->rank != 5 || (p->dims[2] != 3 && p->dims[2] != 4)) {
        return invalid("p must be [X,Y,3 or 4,H,D]");
    }
    const int64_t X = p->dims[0], Y = p->dims[1], G = p->dims[2], H = p->dims[3], D = p->dims[4];
    const int64_t N = column ? Y : X, S = column ? X : Y;
    if (elements(bias) != H * S * S || elements(kmask) != N * S ||
        (G == 4 && elements(gate_bias) != H * D)) {
        return invalid("bias must be [H,S,S], kmask [N,S], gate_bias [H,D]");
    }
    if (elements(out) != X * Y * H * D) return invalid(std::string(what) + ": out must be [X,Y,H,D]");
    if (lims && elements(lims) != N + 1) return invalid("attention_packed_trim: lims must be [N+1]");
    if (!fwd_config_ok(D, block_q, block_k)) return invalid("volta_mma: unsupported (D, bq, bk)");
    if (!aligned16(p->data) || !aligned16(out->data)) {
        return invalid(std::string(what) + ": p and out must be 16-byte aligned");
    }
    if (N * H * S == 0) return ok();
    const half_t* pp = static_cast<const half_t*>(p->data);
    FwdArgs a{};
    const int64_t pn = G * H * D, pr = Y * pn, on = H * D, orow = Y * on;
    if (column) {
        a.qn = pn; a.qh = D; a.qs = pr;
        a.on = on; a.oh = D; a.os = orow;
    } else {
        a.qn = pr; a.qh = D; a.qs = pn;
        a.on = orow; a.oh = D; a.os = on;
    }
    a.kn = a.qn; a.kh = a.qh; a.ks = a.qs;
    a.N = (int)N; a.H = (int)H; a.Sq = (int)S; a.Sk = (int)S; a.D = (int)D;
    a.q = pp;
    a.k = pp + H * D;
    a.v = pp + 2 * H * D;
    a.gate = G == 4 ? pp + 3 * H * D : nullptr;
    a.gate_bias = G == 4 ? static_cast<const half_t*>(gate_bias->data) : nullptr;
    a.lims = lims ? static_cast<const int32_t*>(lims->data) : nullptr;
    a.bias = static_cast<const half_t*>(bias->data);
    a.kmask = static_cast<const uint8_t*>(kmask->data);
    a.out = static_cast<half_t*>(out->data);
    a.lse = nullptr;
    a.scale = scale;
    a.bias_vec = S % 8 == 0 && aligned16(a.bias) && (int64_t)S * S * 2 < ((int64_t)1 << 31);
    a.order = H % 2 == 0 ? kOrderHeadPairs : kOrderRows;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (lims) {
        return G == 4 ? dispatch_fwd<false, true, true>(s, device, a)
                      : dispatch_fwd<false, false, true>(s, device, a);
    }
    return G == 4 ? dispatch_fwd<false, true, false>(s, device, a)
                  : dispatch_fwd<false, false, false>(s, device, a);
}

extern "C" int clk_attention_packed(clk_stream stream, int32_t device, const clk_buffer* p,
                                    const clk_buffer* bias, const clk_buffer* kmask,
                                    const clk_buffer* gate_bias, const clk_buffer* out, float scale,
                                    int64_t block_q, int64_t block_k, int32_t column) {
    return packed_common(stream, device, p, bias, kmask, gate_bias, nullptr, out, scale, block_q,
                         block_k, column);
}

extern "C" int clk_attention_packed_trim(clk_stream stream, int32_t device, const clk_buffer* p,
                                         const clk_buffer* bias, const clk_buffer* kmask,
                                         const clk_buffer* gate_bias, const clk_buffer* lims,
                                         const clk_buffer* out, float scale, int64_t block_q,
                                         int64_t block_k, int32_t column) {
    if (lims == nullptr) return invalid("attention_packed_trim: lims is missing");
    return packed_common(stream, device, p, bias, kmask, gate_bias, lims, out, scale, block_q,
                         block_k, column);
}
