// Q8 A16 projection for many tokens (prefill) on fp16 matrix cores: the
// "mfma" route above the decode kernels' 32 tokens.
//
// out[t][n] = fp16( sum_g D[t][n][g] * ws[n][g] ),  D = sum_{k in g} x[t][k] * code[n][k]
//
// Each 32-column group's D is one v_mfma_f32_16x16x32_f16 on the fp16
// activations and the int8 codes converted to fp16 exactly (every x * code
// product is exact in fp32); the group scale is one fp32 FMA per (t, n, g),
// groups summed in natural order, so outputs agree with the canonical order
// (blocks.cu:306-321) to fp32 association, like the decode route.
//
// Tiling: a workgroup of WM x WN waves computes (WM*TI*16) tokens x
// (WN*TJ*16) rows, each wave TI x TJ tiles of 16 x 16. GS groups are staged at
// a time in two LDS buffers: the tile's activation rows (32 GS halves each)
// and weight rows (32 GS codes converted to fp16 once per workgroup) plus the
// weight scales. Global loads run PF stages ahead in registers; one barrier
// per stage. LDS rows are 4 GS 16-byte units XOR-swizzled by (row >> 1) so
// that 16 consecutive rows' fragment reads fall on distinct banks. The output
// tile leaves through LDS as 16-byte row units.
#include "common.hpp"

#include <algorithm>

namespace vt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Sixteen int8 codes -> sixteen fp16 values, exactly (u = c + 128 as the
// mantissa of 1024 + u, then -1152).
__device__ __forceinline__ void codes16_to_fp16(const uint4 w, uint4& lo, uint4& hi) {
    const half2v bias = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    std::uint32_t h[8];
    const std::uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const std::uint32_t u = words[i] ^ 0x80808080u;
        const half2v a = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x05010400u)) + bias;
        const half2v b = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x05030402u)) + bias;
        h[2 * i] = __builtin_bit_cast(std::uint32_t, a);
        h[2 * i + 1] = __builtin_bit_cast(std::uint32_t, b);
    }
    lo = make_uint4(h[0], h[1], h[2], h[3]);
    hi = make_uint4(h[4], h[5], h[6], h[7]);
}

// XOR swizzle of the 16-byte units of a staged row of U units (4 or 8), so
// that 16 consecutive rows' fragment reads fall on distinct banks.
template <int U>
__device__ __forceinline__ int swizzle(int row) { return (row >> 1) & (U - 1); }

// GS groups of 32 columns per stage.
template <int WM, int WN, int TI, int TJ, int GS>
struct PrefillGeom {
    static constexpr int kThreads = WM * WN * 64;
    static constexpr int kTM = WM * TI * 16;      // tokens per workgroup
    static constexpr int kTN = WN * TJ * 16;      // weight rows per workgroup
    static constexpr int kU = 4 * GS;             // 16-byte fp16 units per staged row
    static constexpr int kAUnits = kTM * kU;      // 16-byte activation loads per stage
    static constexpr int kBUnits = kTN * 2 * GS;  // 16-byte code loads per stage (32 codes a row a group)
    static constexpr int kAPer = (kAUnits + kThreads - 1) / kThreads;
    static constexpr int kBPer = (kBUnits + kThreads - 1) / kThreads;
    static_assert(kAUnits % kThreads == 0 || kAUnits < kThreads, "whole loads per thread");
    static_assert(kBUnits % kThreads == 0 || kBUnits < kThreads, "whole loads per thread");
    static_assert(kTN * GS <= kThreads, "one scale per thread");
};

template <int WM, int WN, int TI, int TJ, int GS>
struct PrefillStage {
    using G = PrefillGeom<WM, WN, TI, TJ, GS>;
    uint4 a[G::kAPer];
    uint4 b[G::kBPer];
    unsigned short ws;
};

template <int WM, int WN, int TI, int TJ, int PF, int GS>
__global__ __launch_bounds__(WM * WN * 64) void q8_prefill(const __half* __restrict__ x,
                                                          const std::int8_t* __restrict__ codes,
                                                          const __half* __restrict__ scales, __half* __restrict__ out,
                                                          int tokens, int n, int k, int padded, int groups) {
    using G = PrefillGeom<WM, WN, TI, TJ, GS>;
    using Stage = PrefillStage<WM, WN, TI, TJ, GS>;
    constexpr int TM = G::kTM, TN = G::kTN, T = G::kThreads, U = G::kU;
    constexpr int kStageBytes = 2 * (TM + TN) * U * 16 + 2 * GS * TN * 4;
    constexpr int kPitch = TN + 8;  // halves per token row of the output tile
    constexpr int kBytes = kStageBytes > TM * kPitch * 2 ? kStageBytes : TM * kPitch * 2;
    __shared__ __attribute__((aligned(16))) unsigned char lds[kBytes];
    auto* a_lds = reinterpret_cast<uint4(*)[TM * U]>(lds);
    auto* b_lds = reinterpret_cast<uint4(*)[TN * U]>(lds + 2 * TM * U * 16);
    auto* ws_lds = reinterpret_cast<float(*)[GS][TN]>(lds + 2 * (TM + TN) * U * 16);
    const int stages = (groups + GS - 1) / GS;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int q = lane >> 4, r = lane & 15;
    const int t0 = blockIdx.y * TM, n0 = blockIdx.x * TN;

    // Stage s covers groups GS*s .. GS*s + GS - 1 (columns 32 GS s ..). Activation
    // load u of a thread: unit i = tid + u*T, token i / U of the tile, columns
    // 8 * (i % U) .. +8 of the stage (zero past k or past the last token: the
    // address is clamped and the value replaced at the store).
    const __half* a_src[G::kAPer];
    int a_col[G::kAPer];
    bool a_row_ok[G::kAPer];
#pragma unroll
    for (int u = 0; u < G::kAPer; ++u) {
        const int i = tid + u * T;
        const int tok = i / U;
        a_row_ok[u] = t0 + tok < tokens;
        a_src[u] = x + static_cast<std::int64_t>(min(t0 + tok, tokens - 1)) * k;
        a_col[u] = 8 * (i % U);
    }
    // Code load u: unit i, row i / (2 GS), code bytes 16 * (i % (2 GS)) of the stage.
    const std::int8_t* b_src[G::kBPer];
#pragma unroll
    for (int u = 0; u < G::kBPer; ++u) {
        const int i = tid + u * T;
        b_src[u] = codes + static_cast<std::int64_t>(min(n0 + min(i / (2 * GS), TN - 1), n - 1)) * padded +
                   16 * (i % (2 * GS));
    }
    // Scale slot sid = T - 1 - tid (staged by the last threads): row sid % TN,
    // group sid / TN of the stage.
    const int sid = T - 1 - tid;
    const int s_grp = sid / TN;
    const __half* ws_src = scales + static_cast<std::int64_t>(min(n0 + sid % TN, n - 1)) * (padded / 32);

    auto load = [&](int st, Stage& s) __attribute__((always_inline)) {
        const int c0 = st * 32 * GS;
#pragma unroll
        for (int u = 0; u < G::kAPer; ++u)
            if (G::kAUnits >= T || tid < G::kAUnits)
                s.a[u] = *reinterpret_cast<const uint4*>(a_src[u] + min(c0 + a_col[u], k - 8));
#pragma unroll
        for (int u = 0; u < G::kBPer; ++u)
            if (G::kBUnits >= T || tid < G::kBUnits)
                s.b[u] = *reinterpret_cast<const uint4*>(b_src[u] + min(c0, padded - 32 * GS));
        s.ws = __half_as_ushort(ws_src[min(st * GS + (s_grp < GS ? s_grp : 0), groups - 1)]);
    };
    auto store = [&](const Stage& s, int st, int buf) __attribute__((always_inline)) {
        const int c0 = st * 32 * GS;
#pragma unroll
        for (int u = 0; u < G::kAPer; ++u) {
            const int i = tid + u * T;
            if (G::kAUnits < T && i >= G::kAUnits) break;
            const int tok = i / U;
            const bool ok = a_row_ok[u] && c0 + a_col[u] < k;  // k % 8 == 0: a unit is all in or all out
            a_lds[buf][tok * U + ((i % U) ^ swizzle<U>(tok))] = ok ? s.a[u] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < G::kBPer; ++u) {
            const int i = tid + u * T;
            if (G::kBUnits < T && i >= G::kBUnits) break;
            const int row = i / (2 * GS), piece = i % (2 * GS);
            uint4 lo, hi;
            codes16_to_fp16(s.b[u], lo, hi);
            b_lds[buf][row * U + ((2 * piece) ^ swizzle<U>(row))] = lo;
            b_lds[buf][row * U + ((2 * piece + 1) ^ swizzle<U>(row))] = hi;
        }
        // A group past the last one (groups % GS != 0) carries scale 0.
        if (sid < TN * GS)
            ws_lds[buf][s_grp][sid % TN] = st * GS + s_grp < groups ? __half2float(__ushort_as_half(s.ws)) : 0.0f;
    };

    float4v y[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) y[i][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    // A stage's fragments, read from LDS before the next stage is converted
    // into the other buffer, so the conversion covers the read latency.
    struct Frag {
        half8 fa[GS][TI];
        half8 fb[GS][TJ];
        float wsv[GS][TJ];
    };
    auto read = [&](int buf, Frag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int gg = 0; gg < GS; ++gg) {
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int row = wn * TJ * 16 + j * 16 + r;
                f.fb[gg][j] = __builtin_bit_cast(half8, b_lds[buf][row * U + ((4 * gg + q) ^ swizzle<U>(row))]);
                f.wsv[gg][j] = ws_lds[buf][gg][row];
            }
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const int tok = wm * TI * 16 + i * 16 + r;
                f.fa[gg][i] = __builtin_bit_cast(half8, a_lds[buf][tok * U + ((4 * gg + q) ^ swizzle<U>(tok))]);
            }
        }
    };
    // Groups in natural order; each tile's MFMA is followed by the scaling of
    // an earlier tile (the schedule below pins the interleave, so the matrix
    // cores run under the wave's own VALU work instead of the epilogue being
    // gathered after the stage's barrier).
    auto math = [&](const Frag& f) __attribute__((always_inline)) {
        const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int gg = 0; gg < GS; ++gg)
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.fa[gg][i], f.fb[gg][j], zero, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) y[i][j][e] = fmaf(d[e], f.wsv[gg][j], y[i][j][e]);
                }
#pragma unroll
        for (int t = 0; t < GS * TI * TJ; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
        }
    };

    // Stage s is loaded PF stages ahead into register stage s % PF, converted
    // into LDS buffer s % 2 while stage s - 1 is multiplied out, and consumed
    // after the barrier that ends that step. Full rounds of PF steps have no
    // branch on the stage index (loads and stores past the last stage are
    // clamped and never consumed); the last partial round is guarded.
    static_assert(PF % 2 == 0, "the buffer parity of a step is fixed within a round");
    Stage st[PF];
#pragma unroll
    for (int s = 0; s < PF; ++s) load(min(s, stages - 1), st[s]);
    store(st[0], 0, 0);
    load(min(PF, stages - 1), st[0]);
    __syncthreads();
    int g0 = 0;
    for (; g0 + PF <= stages; g0 += PF) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
            Frag f;
            read(s & 1, f);
            const int nxt = min(g0 + s + 1, stages - 1);
            store(st[(s + 1) % PF], nxt, (s + 1) & 1);
            load(min(g0 + s + 1 + PF, stages - 1), st[(s + 1) % PF]);
            math(f);
            __syncthreads();
        }
    }
    if (g0 < stages) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
            if (g0 + s < stages) {
                Frag f;
                read(s & 1, f);
                store(st[(s + 1) % PF], min(g0 + s + 1, stages - 1), (s + 1) & 1);
                math(f);
                __syncthreads();
            }
        }
    }

    // Output tile: fp16 through LDS (token rows padded by 8 halves so the four
    // token quads of a wave's 2-byte writes fall on distinct banks), then
    // 16-byte row units to HBM.
    auto* o_lds = reinterpret_cast<__half*>(lds);
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o_lds[(wm * TI * 16 + i * 16 + 4 * q + e) * kPitch + wn * TJ * 16 + j * 16 + r] =
                    from_f32<__half>(y[i][j][e]);
    __syncthreads();
    const bool vec = (n % 8) == 0 && (reinterpret_cast<std::uintptr_t>(out) & 15) == 0;
    constexpr int kUnits = TM * TN / 8;
#pragma unroll
    for (int u = tid; u < kUnits; u += T) {
        const int tok = u / (TN / 8), c = (u % (TN / 8)) * 8;
        const int t = t0 + tok, col = n0 + c;
        if (t >= tokens || col >= n) continue;
        const __half* src = o_lds + tok * kPitch + c;
        __half* dst = out + static_cast<std::int64_t>(t) * n + col;
        if (vec) {
            *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
        } else {
            for (int e = 0; e < 8 && col + e < n; ++e) dst[e] = src[e];
        }
    }
}

template <int WM, int WN, int TI, int TJ, int PF, int GS = 1>
void launch_prefill(const __half* x, const std::int8_t* codes, const __half* scales, __half* out, int tokens, int n,
                    int k, int padded, hipStream_t stream) {
    using G = PrefillGeom<WM, WN, TI, TJ, GS>;
    const int groups = (k + 31) / 32;
    const dim3 grid((n + G::kTN - 1) / G::kTN, (tokens + G::kTM - 1) / G::kTM);
    require(grid.y <= 65535, "token tiles exceed the launch grid");
    q8_prefill<WM, WN, TI, TJ, PF, GS><<<grid, G::kThreads, 0, stream>>>(x, codes, scales, out, tokens, n, k,
                                                                        padded, groups);
}

// The exact two-term fp16 form of Q8 weights, for the dense route: row j of
// the shadow holds hi = fp16(q*s) in columns [0, k) and lo = q*s - hi in
// [k, 2k). q*s is exact in fp32 (an 8-bit integer times an 11-bit
// significand), hi is its RNE fp16 rounding, and the difference is a multiple
// of the scale's ulp smaller than half an ulp of hi, at most 8 significant
// bits, which fp16 (with its subnormals) holds exactly; so hi + lo == q*s for
// every scale below 516. At 516 and above 127*s rounds past 65504: hi becomes
// inf and lo -inf, and every output that row touches is NaN, never a finite
// wrong value. Thread: 8 columns of one row (k % 8 == 0).
__global__ __launch_bounds__(256) void q8_split(const std::int8_t* __restrict__ codes, const __half* __restrict__ scales,
                                                __half* __restrict__ shadow, int row0, int k, int padded) {
    const int c = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (c >= k) return;
    const std::int64_t row = row0 + static_cast<std::int64_t>(blockIdx.y);
    const uint2 w = *reinterpret_cast<const uint2*>(codes + row * padded + c);
    const float s = __half2float(scales[row * (padded / 32) + c / 32]);
    const std::uint32_t words[2] = {w.x, w.y};
    std::uint32_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        float v[2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
            v[j] = static_cast<float>(static_cast<std::int8_t>(words[(i + j) / 4] >> (8 * ((i + j) % 4)))) * s;
        const __half h0 = __float2half_rn(v[0]), h1 = __float2half_rn(v[1]);
        const __half l0 = __float2half_rn(v[0] - __half2float(h0)), l1 = __float2half_rn(v[1] - __half2float(h1));
        hi[i / 2] = static_cast<std::uint32_t>(__half_as_ushort(h0)) | static_cast<std::uint32_t>(__half_as_ushort(h1)) << 16;
        lo[i / 2] = static_cast<std::uint32_t>(__half_as_ushort(l0)) | static_cast<std::uint32_t>(__half_as_ushort(l1)) << 16;
    }
    __half* dst = shadow + static_cast<std::int64_t>(blockIdx.y) * 2 * k + c;
    *reinterpret_cast<uint4*>(dst) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *reinterpret_cast<uint4*>(dst + k) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
}

// x [tokens][k] -> x2 [tokens][2k] = [x | x] (the activations of the dense
// route's doubled K). Thread: 8 halves (k % 8 == 0).
__global__ __launch_bounds__(256) void q8_dup_rows(const __half* __restrict__ x, __half* __restrict__ x2, int k) {
    const int c = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (c >= k) return;
    const std::int64_t t = blockIdx.y;
    const uint4 v = *reinterpret_cast<const uint4*>(x + t * k + c);
    *reinterpret_cast<uint4*>(x2 + t * 2 * k + c) = v;
    *reinterpret_cast<uint4*>(x2 + t * 2 * k + k + c) = v;
}

}  // namespace

void q8_split_launch(const std::int8_t* codes, const __half* scales, void* shadow, int row0, int rows, int k,
                     int padded, hipStream_t stream) {
    require(k % 8 == 0 && rows > 0 && rows <= 65535 && padded == padded_k(k), "invalid Q8 split geometry");
    require(aligned(codes, 8) && aligned(scales, 2) && aligned(shadow, 16), "misaligned Q8 split operand");
    q8_split<<<dim3((k / 8 + 255) / 256, rows), 256, 0, stream>>>(codes, scales, static_cast<__half*>(shadow), row0, k,
                                                                 padded);
}

void q8_dup_launch(const void* x, void* x2, int tokens, int k, hipStream_t stream) {
    require(k % 8 == 0 && tokens > 0 && tokens <= 65535, "invalid activation geometry for the dense Q8 route");
    q8_dup_rows<<<dim3((k / 8 + 255) / 256, tokens), 256, 0, stream>>>(static_cast<const __half*>(x),
                                                                       static_cast<__half*>(x2), k);
}

void q8_prefill_launch(const void* x, const std::int8_t* codes, const __half* scales, void* out, int tokens, int n,
                       int k, int padded, int dtype, hipStream_t stream) {
    require(x && codes && scales && out, "null Q8 operand");
    require(tokens > 0 && n > 0 && k > 0 && padded == padded_k(k), "invalid Q8 geometry");
    require(static_cast<std::int64_t>(tokens) * n < INT32_MAX, "Q8 output count exceeds int32");
    require(dtype == kF16, "the Q8 prefill GEMM takes FP16 activations");
    require(k % 8 == 0 && aligned(x, 16), "the Q8 prefill GEMM needs k % 8 == 0 and 16-byte aligned x");
    require(aligned(codes, 16) && aligned(scales, 2) && aligned(out, 2), "misaligned Q8 operand");
    // Four tilings of 8 waves: 256 x 128 (waves of 64 x 64), 128 x 160
    // (32 x 80), 128 x 224 (32 x 112), each one workgroup per CU, and
    // 128 x 128 with two groups per stage (the small grids' tiling). The
    // launch takes the one with the least time over whole tile rounds on the
    // CUs, from their measured rates per unit of work (1 : 0.76 : 0.89 :
    // 0.80): small grids take 128 x 128 as before; at M = 2048,
    // 7168 rows take 128 x 224 (512 tiles, two rounds), 5120 rows 128 x 160
    // (512 tiles), 34816 rows 256 x 128 (config-2 W8A16 QKV / o_proj / gate+up
    // / down 303 / 306 / 1225 / 818 -> 297 / 256 / 1225 / 685 us; same bits
    // in every tiling, the groups being summed in natural order).
    const auto* xp = static_cast<const __half*>(x);
    auto* op = static_cast<__half*>(out);
    constexpr GemmTiling kTilings[4] = {{256, 128, 1.0}, {128, 160, 0.76}, {128, 224, 0.89}, {128, 128, 0.80}};
    const int best = pick_tiling(tokens, n, kTilings);
    if (best == 0) launch_prefill<4, 2, 4, 4, 2, 1>(xp, codes, scales, op, tokens, n, k, padded, stream);
    else if (best == 1) launch_prefill<4, 2, 2, 5, 2, 1>(xp, codes, scales, op, tokens, n, k, padded, stream);
    else if (best == 2) launch_prefill<4, 2, 2, 7, 2, 1>(xp, codes, scales, op, tokens, n, k, padded, stream);
    else launch_prefill<2, 4, 4, 2, 2, 2>(xp, codes, scales, op, tokens, n, k, padded, stream);
}

}  // namespace vt

// Extension: the Q8 A16 projection for many tokens on fp16 matrix cores (same
// arguments as venturi_q8_head_run; fp16 activations, k % 8 == 0, any token
// count; intended for prefill, M >= 33).
extern "C" __attribute__((visibility("default"))) int venturi_q8_prefill_run(const void* x, const std::int8_t* codes,
                                                                            const __half* scales, void* out,
                                                                            int tokens, int n, int k, int padded,
                                                                            int dtype, void* stream) {
    return vt::guarded([&] {
        vt::q8_prefill_launch(x, codes, scales, out, tokens, n, k, padded, dtype, static_cast<hipStream_t>(stream));
    });
}
