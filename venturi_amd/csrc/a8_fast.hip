// W8A8 projection for many tokens on matrix cores with a free fp32 order
// (the "mfma" A8 route).
//
// out[t][n] = fp16( sum_g d[t][n][g] * (ws[n][g] * as[t][g]) )   (one pass)
//
// d is the exact integer dot of the group's 32 activation and weight codes:
// int8 codes are exact in fp16, every product of two codes is an integer
// below 2^14 and every partial sum of 32 of them an integer below 2^19, so
// v_mfma_f32_16x16x32_f16 returns d exactly as fp32 (the int32 accumulator
// of the reference, q8_dp4a.cuh:47-58). The group scaling is the reference's
// (one fp32 product ws*as, one FMA), but groups are accumulated in natural
// order into one fp32 sum per output instead of the reference's 32 lane
// slots and shuffle tree (q8_dp4a.cuh:59-70), so outputs agree with the
// reference to fp32 association, not bit for bit. With two passes (the
// residual profile) the group term is (d0 * as0 + d1 * as1) * ws.
//
// Tiling: a workgroup of WM x WN waves computes (WM*TI*16) tokens x
// (WN*TJ*16) rows; each wave computes TI x TJ MFMA tiles of 16 x 16. Groups
// are staged one at a time in two LDS buffers: the group's codes (converted
// to fp16 once per workgroup) and scales. Global loads run two groups ahead
// in registers; one barrier per group. LDS rows are 32 halves (four 16-byte
// units) with the units of row t XOR-swizzled by (t >> 1) & 3, so the
// 16-byte fragment reads of 16 consecutive rows fall on distinct banks. The
// output tile leaves through LDS as 16-byte row units.
#include "common.hpp"

#include <algorithm>
#include <utility>

namespace vt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

// Sixteen int8 codes -> sixteen fp16 values, exactly (u = c + 128 as the
// mantissa of 1024 + u, then -1152).
__device__ __forceinline__ void codes16_to_half(const uint4 w, uint4& lo, uint4& hi) {
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
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

__device__ __forceinline__ int swz(int row) { return (row >> 1) & 3; }

template <int P, int WM, int WN, int TI, int TJ>
struct FastGeom {
    static constexpr int kThreads = WM * WN * 64;
    static constexpr int kTM = WM * TI * 16;  // tokens per workgroup
    static constexpr int kTN = WN * TJ * 16;  // rows per workgroup
    static constexpr int kAUnits = P * kTM * 2;  // 16-byte code loads per group (activations)
    static constexpr int kBUnits = kTN * 2;      // 16-byte code loads per group (weights)
    static constexpr int kAPer = (kAUnits + kThreads - 1) / kThreads;
    static constexpr int kBPer = (kBUnits + kThreads - 1) / kThreads;
    static_assert(kAUnits % kThreads == 0 || kAUnits < kThreads, "whole loads per thread");
    static_assert(kBUnits % kThreads == 0 || kBUnits < kThreads, "whole loads per thread");
    static_assert(P * kTM <= kThreads && kTN <= kThreads, "one scale per thread");
};

template <int P, int WM, int WN, int TI, int TJ>
struct FastStage {
    using G = FastGeom<P, WM, WN, TI, TJ>;
    uint4 a[G::kAPer];
    uint4 b[G::kBPer];
    float as;
    unsigned short ws;
};

template <int P, int WM, int WN, int TI, int TJ>
struct FastLds {
    using G = FastGeom<P, WM, WN, TI, TJ>;
    static constexpr int kA = P * G::kTM * 4;   // 16-byte units of one activation buffer
    static constexpr int kB = G::kTN * 4;       // 16-byte units of one weight buffer
    static constexpr int kStage = 2 * (kA + kB) * 16 + 2 * (P * G::kTM + G::kTN) * 4;
    static constexpr int kPitch = G::kTN + 8;   // halves per token row of the output tile
    static constexpr int kOut = G::kTM * kPitch * 2;
    static constexpr int kBytes = kStage > kOut ? kStage : kOut;
};

template <int P, int WM, int WN, int TI, int TJ>
__global__ __launch_bounds__(WM * WN * 64) void a8_gemm_fast(const std::int8_t* __restrict__ acodes,
                                                            const float* __restrict__ ascales,
                                                            const std::int8_t* __restrict__ wcodes,
                                                            const __half* __restrict__ wscales,
                                                            __half* __restrict__ out, int tokens, int n, int padded,
                                                            int groups) {
    using G = FastGeom<P, WM, WN, TI, TJ>;
    using L = FastLds<P, WM, WN, TI, TJ>;
    using Stage = FastStage<P, WM, WN, TI, TJ>;
    constexpr int TM = G::kTM, TN = G::kTN, T = G::kThreads;
    __shared__ __attribute__((aligned(16))) unsigned char lds[L::kBytes];
    auto* a_lds = reinterpret_cast<uint4(*)[L::kA]>(lds);
    auto* b_lds = reinterpret_cast<uint4(*)[L::kB]>(lds + 2 * L::kA * 16);
    auto* as_lds = reinterpret_cast<float(*)[P * TM]>(lds + 2 * (L::kA + L::kB) * 16);
    auto* ws_lds = reinterpret_cast<float(*)[TN]>(lds + 2 * (L::kA + L::kB) * 16 + 2 * P * TM * 4);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int q = lane >> 4, r = lane & 15;
    const int t0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;

    // Staging sources. Activation load u of a thread: unit i = tid + u*T,
    // pass i / (2*TM), token (i / 2) % TM, half i % 2 of the group's 32 bytes.
    const std::int8_t* a_src[G::kAPer];
#pragma unroll
    for (int u = 0; u < G::kAPer; ++u) {
        const int i = tid + u * T;
        const int p = i / (2 * TM), tok = (i / 2) % TM;
        a_src[u] = acodes + (min(p, P - 1) * count + static_cast<std::int64_t>(min(t0 + tok, tokens - 1)) * groups) * 32 +
                   16 * (i & 1);
    }
    const std::int8_t* b_src[G::kBPer];
#pragma unroll
    for (int u = 0; u < G::kBPer; ++u) {
        const int i = tid + u * T;
        b_src[u] = wcodes + static_cast<std::int64_t>(min(n0 + min(i / 2, TN - 1), n - 1)) * padded + 16 * (i & 1);
    }
    // Scales are staged by the last threads of the workgroup (the weight codes,
    // fewer than the activation codes, are staged by the first ones).
    const int sid = T - 1 - tid;
    const int s_pass = min(sid / TM, P - 1);
    const float* as_src =
        ascales + s_pass * count + static_cast<std::int64_t>(min(t0 + sid % TM, tokens - 1)) * groups;
    const __half* ws_src = wscales + static_cast<std::int64_t>(min(n0 + sid % TN, n - 1)) * (padded / 32);

    // Group g's operands into registers (g is clamped by the caller, so a load
    // past the last group re-reads it and is never consumed).
    auto load = [&](int g, Stage& s) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < G::kAPer; ++u)
            if (G::kAUnits >= T || tid < G::kAUnits) s.a[u] = *reinterpret_cast<const uint4*>(a_src[u] + g * 32);
#pragma unroll
        for (int u = 0; u < G::kBPer; ++u)
            if (G::kBUnits >= T || tid < G::kBUnits) s.b[u] = *reinterpret_cast<const uint4*>(b_src[u] + g * 32);
        s.as = as_src[g];
        s.ws = __half_as_ushort(ws_src[g]);
    };
    auto store = [&](const Stage& s, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < G::kAPer; ++u) {
            const int i = tid + u * T;
            if (G::kAUnits < T && i >= G::kAUnits) break;
            const int row = i / 2;  // pass-major row p*TM + token
            const int tok = row % TM;
            uint4 lo, hi;
            codes16_to_half(s.a[u], lo, hi);
            a_lds[buf][row * 4 + ((2 * (i & 1)) ^ swz(tok))] = lo;
            a_lds[buf][row * 4 + ((2 * (i & 1) + 1) ^ swz(tok))] = hi;
        }
#pragma unroll
        for (int u = 0; u < G::kBPer; ++u) {
            const int i = tid + u * T;
            if (G::kBUnits < T && i >= G::kBUnits) break;
            const int row = i / 2;
            uint4 lo, hi;
            codes16_to_half(s.b[u], lo, hi);
            b_lds[buf][row * 4 + ((2 * (i & 1)) ^ swz(row))] = lo;
            b_lds[buf][row * 4 + ((2 * (i & 1) + 1) ^ swz(row))] = hi;
        }
        if (sid < P * TM) as_lds[buf][sid] = s.as;
        if (sid < TN) ws_lds[buf][sid] = __half2float(__ushort_as_half(s.ws));
    };

    float4v y[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) y[i][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    struct Frag {
        half8 fa[P][TI];
        half8 fb[TJ];
        float4 asv[P][TI];
        float wsv[TJ];
    };
    auto read = [&](int buf, Frag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int row = wn * TJ * 16 + j * 16 + r;
            f.fb[j] = __builtin_bit_cast(half8, b_lds[buf][row * 4 + (q ^ swz(row))]);
            f.wsv[j] = ws_lds[buf][row];
        }
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            const int tok = wm * TI * 16 + i * 16 + r;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                f.fa[p][i] = __builtin_bit_cast(half8, a_lds[buf][(p * TM + tok) * 4 + (q ^ swz(tok))]);
                f.asv[p][i] = *reinterpret_cast<const float4*>(&as_lds[buf][p * TM + wm * TI * 16 + i * 16 + 4 * q]);
            }
        }
    };
    // One group: each tile's MFMA is followed by the scaling of an earlier
    // tile, so one wave's matrix-core work runs under its own VALU epilogue
    // (the schedule below pins that interleave: the epilogue may not be
    // gathered after the group's barrier, where both waves of a SIMD would
    // run their VALU work at once).
    constexpr int kEpi = P == 1 ? 8 : 12;  // VALU instructions per tile
    auto math = [&](const Frag& f) __attribute__((always_inline)) {
        const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                if constexpr (P == 1) {
                    const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.fa[0][i], f.fb[j], zero, 0, 0, 0);
                    const float a4[4] = {f.asv[0][i].x, f.asv[0][i].y, f.asv[0][i].z, f.asv[0][i].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) y[i][j][e] = fmaf(d[e], f.wsv[j] * a4[e], y[i][j][e]);
                } else {
                    const float4v d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.fa[0][i], f.fb[j], zero, 0, 0, 0);
                    const float4v d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.fa[1][i], f.fb[j], zero, 0, 0, 0);
                    const float a0[4] = {f.asv[0][i].x, f.asv[0][i].y, f.asv[0][i].z, f.asv[0][i].w};
                    const float a1[4] = {f.asv[1][i].x, f.asv[1][i].y, f.asv[1][i].z, f.asv[1][i].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float t = fmaf(d1[e], a1[e], d0[e] * a0[e]);
                        y[i][j][e] = fmaf(t, f.wsv[j], y[i][j][e]);
                    }
                }
            }
#pragma unroll
        for (int t = 0; t < TI * TJ; ++t) {
            __builtin_amdgcn_sched_group_barrier(0x008, P, 0);     // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, kEpi, 0);  // VALU
        }
    };

    // Pipeline over groups, two LDS buffers and two register stages: while
    // group g is multiplied out of buffer g % 2, group g + 1 (loaded two
    // groups earlier) is converted into the other buffer and group g + 3 is
    // requested; one barrier per group. The body of a step has no branches
    // on g, so the scheduler sees the fragment reads, the conversion and the
    // interleaved MFMA / VALU work as one region.
    Stage st0, st1;
    load(0, st0);
    load(min(1, groups - 1), st1);
    store(st0, 0);
    load(min(2, groups - 1), st0);
    __syncthreads();
    int g = 0;
    for (; g + 1 < groups; g += 2) {
        Frag f;
        read(0, f);
        store(st1, 1);
        load(min(g + 3, groups - 1), st1);
        math(f);
        __syncthreads();
        read(1, f);
        store(st0, 0);
        load(min(g + 4, groups - 1), st0);
        math(f);
        __syncthreads();
    }
    if (g < groups) {
        Frag f;
        read(0, f);
        math(f);
        __syncthreads();
    }

    // Output tile: fp16 through LDS (token rows of TN halves, padded by 8 so
    // the four token quads of a wave's 2-byte writes fall on distinct banks),
    // then 16-byte row units to HBM.
    auto* o_lds = reinterpret_cast<__half*>(lds);
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o_lds[(wm * TI * 16 + i * 16 + 4 * q + e) * L::kPitch + wn * TJ * 16 + j * 16 + r] =
                    from_f32<__half>(y[i][j][e]);
    __syncthreads();
    const bool vec = (n % 8) == 0 && (reinterpret_cast<std::uintptr_t>(out) & 15) == 0;
    constexpr int kUnits = TM * TN / 8;
#pragma unroll
    for (int u = tid; u < kUnits; u += T) {
        const int tok = u / (TN / 8), c = (u % (TN / 8)) * 8;
        const int t = t0 + tok, col = n0 + c;
        if (t >= tokens || col >= n) continue;
        const __half* src = o_lds + tok * L::kPitch + c;
        __half* dst = out + static_cast<std::int64_t>(t) * n + col;
        if (vec) {
            *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(src);
        } else {
            for (int e = 0; e < 8 && col + e < n; ++e) dst[e] = src[e];
        }
    }
}

template <int P, int WM, int WN, int TI, int TJ>
void launch_fast(const std::int8_t* acodes, const float* ascales, const std::int8_t* codes, const __half* scales,
                 __half* out, int tokens, int n, int padded, int groups, hipStream_t stream) {
    using G = FastGeom<P, WM, WN, TI, TJ>;
    const dim3 grid((n + G::kTN - 1) / G::kTN, (tokens + G::kTM - 1) / G::kTM);
    require(grid.y <= 65535, "token tiles exceed the launch grid");
    a8_gemm_fast<P, WM, WN, TI, TJ><<<grid, G::kThreads, 0, stream>>>(acodes, ascales, codes, scales, out, tokens, n,
                                                                     padded, groups);
}

}  // namespace

void a8_fast_launch(const void* workspace, const std::int8_t* codes, const __half* scales, void* out, int tokens, int n,
                    int k, int padded, int passes, hipStream_t stream) {
    const int groups = (k + 31) / 32;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const auto* acodes = static_cast<const std::int8_t*>(workspace);
    const auto* ascales = reinterpret_cast<const float*>(acodes + count * 32 * passes);
    auto* y = static_cast<__half*>(out);
    if (passes == 2) {
        launch_fast<2, 4, 2, 2, 4>(acodes, ascales, codes, scales, y, tokens, n, padded, groups, stream);
        return;
    }
    // One pass: 256 x 128, 128 x 160 or 128 x 224 tiles (waves of 64 x 64,
    // 32 x 80, 32 x 112), whichever leaves the fewest tile rounds on the CUs
    // at the measured rates (config 3 at M = 2048 on MI355X: QKV / o_proj /
    // gate+up / down 457 / 435 / 1781 / 1162 -> 408 / 389 / 1781 / 1038 us;
    // same bits in every tiling, the groups being summed in natural order).
    constexpr GemmTiling kTilings[3] = {{256, 128, 1.0}, {128, 160, 0.76}, {128, 224, 0.89}};
    const int best = pick_tiling(tokens, n, kTilings);
    if (best == 0) launch_fast<1, 4, 2, 4, 4>(acodes, ascales, codes, scales, y, tokens, n, padded, groups, stream);
    else if (best == 1) launch_fast<1, 4, 2, 2, 5>(acodes, ascales, codes, scales, y, tokens, n, padded, groups, stream);
    else launch_fast<1, 4, 2, 2, 7>(acodes, ascales, codes, scales, y, tokens, n, padded, groups, stream);
}

}  // namespace vt
