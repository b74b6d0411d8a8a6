// W8A8 projection for many tokens on matrix cores, bit-exact to the
// reference's per-output order (q8_dp4a.cuh:36-70).
//
// Reference order for output (t, n): 32 lane slots; slot l accumulates, for
// groups g = l, l+32, ... < G and passes p in order,
//     s_l = fmaf(f32(d[t][n][g][p]), ws[n][g] * as[p][t][g], s_l)
// with d the exact int32 dot of the group's 32 codes; the 32 slot sums are
// then reduced by a shfl_down 16/8/4/2/1 tree and rounded to fp16.
//
// Group dots: the int8 codes are exact in fp16, every product of two codes is
// an integer below 2^14 and every partial sum of 32 of them an integer below
// 2^19, so v_mfma_f32_16x16x32_f16 returns d exactly, already as fp32. The
// epilogue per output and group is then one fp32 multiply (ws * as) and one
// FMA, the reference's two roundings.
//
// Tree: slots are visited in the order slot = bitreverse5(position), so the
// pairs of every tree level complete consecutively. One accumulator per level
// takes the first member of its pair and adds the second, which reproduces
// the tree's additions exactly with 5 + 1 registers per output.
//
// Tiling: a 512-thread workgroup computes 128 tokens x 64 rows; wave
// (wm, wn) in 4 x 2 computes 32 x 32 as 2 x 2 MFMA tiles of 16 x 16. Every
// (slot, group) step stages the tile's codes (converted to fp16) and scales in
// LDS; the next step's global loads are in flight while a step computes.
#include "common.hpp"

#include <algorithm>

namespace vt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kTokTile = 128;
constexpr int kRowTile = 64;
constexpr int kRowHalves = 40;  // LDS row: 32 fp16 + 8 pad (80 bytes: conflict-free 16-byte reads)
constexpr int kBatch = 4;       // groups of one slot staged per step

__device__ __forceinline__ int bitrev5(int p) {
    return ((p & 1) << 4) | ((p & 2) << 2) | (p & 4) | ((p & 8) >> 2) | ((p & 16) >> 4);
}

// Four int8 codes -> four fp16 values, exactly (u = c + 128 as the mantissa of 1024 + u).
__device__ __forceinline__ uint2 codes4_to_half(std::uint32_t w) {
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    const std::uint32_t u = w ^ 0x80808080u;
    const half2v bias = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    const half2v lo = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x05010400u)) + bias;
    const half2v hi = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x05030402u)) + bias;
    return make_uint2(__builtin_bit_cast(std::uint32_t, lo), __builtin_bit_cast(std::uint32_t, hi));
}

template <int P>
__global__ __launch_bounds__(512) void a8_gemm(const std::int8_t* __restrict__ acodes,
                                               const float* __restrict__ ascales,
                                               const std::int8_t* __restrict__ wcodes,
                                               const __half* __restrict__ wscales, __half* __restrict__ out,
                                               int tokens, int n, int padded, int groups) {
    // One step stages up to kBatch groups of one slot (g = slot + 32 (kBatch b + j)).
    __shared__ __attribute__((aligned(16))) _Float16 af[P][kTokTile * kBatch * kRowHalves];
    __shared__ __attribute__((aligned(16))) _Float16 bf[kRowTile * kBatch * kRowHalves];
    __shared__ __attribute__((aligned(16))) float as_lds[P][kBatch][kTokTile];
    __shared__ float ws_lds[kBatch][kRowTile];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int q = lane >> 4, r = lane & 15;
    const int t0 = blockIdx.y * kTokTile, n0 = blockIdx.x * kRowTile;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;

    // Staging assignment (clamped rows are computed and never stored; groups past
    // the slot's last are clamped to it and never used):
    // activation codes: token tid / 4, bytes 8 * (tid % 4) of every batched group;
    // weight codes: row tid / 8, bytes 4 * (tid % 8); activation scale: token
    // tid % 128 of batched group tid / 128; weight scale: row tid % 64 of group
    // (tid / 64) % kBatch.
    const std::int64_t a_tok = min(t0 + (tid >> 2), tokens - 1);
    const std::int8_t* a_src[P];
#pragma unroll
    for (int p = 0; p < P; ++p) a_src[p] = acodes + ((p * count) + a_tok * groups) * 32 + 8 * (tid & 3);
    const std::int8_t* b_src = wcodes + static_cast<std::int64_t>(min(n0 + (tid >> 3), n - 1)) * padded + 4 * (tid & 7);
    static_assert(kBatch == 4, "the staging assignment assumes four groups per step");
    const int s_group = tid >> 7;  // 0..3
    const int w_group = (tid >> 6) & (kBatch - 1);
    const float* as_src[P];
#pragma unroll
    for (int p = 0; p < P; ++p)
        as_src[p] = ascales + p * count + static_cast<std::int64_t>(min(t0 + (tid & 127), tokens - 1)) * groups;
    const __half* ws_src = wscales + static_cast<std::int64_t>(min(n0 + (tid & 63), n - 1)) * (padded / 32);

    struct Stage {
        uint2 a[P][kBatch];
        std::uint32_t b[kBatch];
        float as[P];
        unsigned short ws;
    };
    // Groups of a step: g(j) = first + 32 j for j < kBatch, clamped to `last`.
    auto load = [&](int first, int last, Stage& st) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const int g = min(first + 32 * j, last);
#pragma unroll
            for (int p = 0; p < P; ++p) st.a[p][j] = *reinterpret_cast<const uint2*>(a_src[p] + g * 32);
            st.b[j] = *reinterpret_cast<const std::uint32_t*>(b_src + g * 32);
        }
        const int gs = min(first + 32 * s_group, last), gw = min(first + 32 * w_group, last);
#pragma unroll
        for (int p = 0; p < P; ++p) st.as[p] = as_src[p][gs];
        st.ws = __half_as_ushort(ws_src[gw]);
    };
    auto store = [&](const Stage& st) {
        const int tok = tid >> 2;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint2 lo = codes4_to_half(st.a[p][j].x), hi = codes4_to_half(st.a[p][j].y);
                *reinterpret_cast<uint4*>(&af[p][(tok * kBatch + j) * kRowHalves + 8 * (tid & 3)]) =
                    make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
            *reinterpret_cast<uint2*>(&bf[((tid >> 3) * kBatch + j) * kRowHalves + 4 * (tid & 7)]) =
                codes4_to_half(st.b[j]);
        }
#pragma unroll
        for (int p = 0; p < P; ++p) as_lds[p][s_group][tid & 127] = st.as[p];
        if (tid < kBatch * kRowTile) ws_lds[w_group][tid & 63] = __half2float(__ushort_as_half(st.ws));
    };

    // The schedule: position p visits slot bitrev5(p); its groups
    // slot, slot + 32, ... < groups are processed kBatch at a time.
    auto slot_groups = [&](int p) {
        const int slot = bitrev5(p);
        return slot < groups ? (groups - slot + 31) / 32 : 0;
    };
    auto first_position = [&](int p) {  // first position at or after p with groups
        while (p < 32 && slot_groups(p) == 0) ++p;
        return p;
    };
    auto last_group = [&](int p) { return bitrev5(p) + 32 * (slot_groups(p) - 1); };

    float s[16], lv[5][16];
#pragma unroll
    for (int o = 0; o < 16; ++o) s[o] = 0.0f;

    Stage st;
    int next_p = first_position(0), next_b = 0;
    if (next_p < 32) load(bitrev5(next_p), last_group(next_p), st);
    for (int p = 0; p < 32; ++p) {
        const int cnt = slot_groups(p);
        for (int b0 = 0; b0 < cnt; b0 += kBatch) {
            const int live = min(kBatch, cnt - b0);
            __syncthreads();
            store(st);
            __syncthreads();
            // Advance the schedule and prefetch the next step's operands.
            next_b += kBatch;
            if (next_b >= slot_groups(next_p)) {
                next_p = first_position(next_p + 1);
                next_b = 0;
            }
            if (next_p < 32) load(bitrev5(next_p) + 32 * next_b, last_group(next_p), st);

            float wsv[kBatch][2];
#pragma unroll
            for (int j = 0; j < kBatch; ++j)
#pragma unroll
                for (int b = 0; b < 2; ++b) wsv[j][b] = ws_lds[j][wn * 32 + 16 * b + r];
            const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                if (j >= live) break;  // groups in increasing order within the slot
                half8 bfr[2];
#pragma unroll
                for (int b = 0; b < 2; ++b)
                    bfr[b] = *reinterpret_cast<const half8*>(&bf[((wn * 32 + 16 * b + r) * kBatch + j) * kRowHalves + 8 * q]);
#pragma unroll
                for (int p2 = 0; p2 < P; ++p2) {
#pragma unroll
                    for (int a = 0; a < 2; ++a) {
                        const half8 afr =
                            *reinterpret_cast<const half8*>(&af[p2][((wm * 32 + 16 * a + r) * kBatch + j) * kRowHalves + 8 * q]);
                        const float4 as4 = *reinterpret_cast<const float4*>(&as_lds[p2][j][wm * 32 + 16 * a + 4 * q]);
                        const float asv[4] = {as4.x, as4.y, as4.z, as4.w};
#pragma unroll
                        for (int b = 0; b < 2; ++b) {
                            const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(afr, bfr[b], zero, 0, 0, 0);
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                float& acc = s[(a * 2 + b) * 4 + e];
                                acc = __fmaf_rn(d[e], __fmul_rn(wsv[j][b], asv[e]), acc);
                            }
                        }
                    }
                }
            }
        }
        // Fold slot bitrev5(p) into the level accumulators: a level takes the
        // first member of its pair and adds the second (position bits h0..h4).
        const int h0 = p & 1, h1 = (p >> 1) & 1, h2 = (p >> 2) & 1, h3 = (p >> 3) & 1, h4 = (p >> 4) & 1;
#pragma unroll
        for (int o = 0; o < 16; ++o) lv[0][o] = h0 ? lv[0][o] + s[o] : s[o];
        if (h0) {
#pragma unroll
            for (int o = 0; o < 16; ++o) lv[1][o] = h1 ? lv[1][o] + lv[0][o] : lv[0][o];
            if (h1) {
#pragma unroll
                for (int o = 0; o < 16; ++o) lv[2][o] = h2 ? lv[2][o] + lv[1][o] : lv[1][o];
                if (h2) {
#pragma unroll
                    for (int o = 0; o < 16; ++o) lv[3][o] = h3 ? lv[3][o] + lv[2][o] : lv[2][o];
                    if (h3) {
#pragma unroll
                        for (int o = 0; o < 16; ++o) lv[4][o] = h4 ? lv[4][o] + lv[3][o] : lv[3][o];
                    }
                }
            }
        }
#pragma unroll
        for (int o = 0; o < 16; ++o) s[o] = 0.0f;
    }

#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int row = n0 + wn * 32 + b * 16 + r;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = t0 + wm * 32 + a * 16 + 4 * q + e;
                if (t < tokens && row < n)
                    out[static_cast<std::int64_t>(t) * n + row] = from_f32<__half>(lv[4][(a * 2 + b) * 4 + e]);
            }
        }
}

}  // namespace

void a8_gemm_launch(const void* workspace, const std::int8_t* codes, const __half* scales, void* out, int tokens,
                    int n, int k, int padded, int passes, hipStream_t stream) {
    const int groups = (k + 31) / 32;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const auto* acodes = static_cast<const std::int8_t*>(workspace);
    const auto* ascales = reinterpret_cast<const float*>(acodes + count * 32 * passes);
    const dim3 grid((n + kRowTile - 1) / kRowTile, (tokens + kTokTile - 1) / kTokTile);
    require(grid.y <= 65535, "token tiles exceed the launch grid");
    if (passes == 1)
        a8_gemm<1><<<grid, 512, 0, stream>>>(acodes, ascales, codes, scales, static_cast<__half*>(out), tokens, n,
                                              padded, groups);
    else
        a8_gemm<2><<<grid, 512, 0, stream>>>(acodes, ascales, codes, scales, static_cast<__half*>(out), tokens, n,
                                              padded, groups);
}

}  // namespace vt
