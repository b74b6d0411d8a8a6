// W8A8 projection for many tokens on int8 matrix cores, bit-exact to the
// reference's per-output order (q8_dp4a.cuh:36-70).
//
// Reference order for output (t, n): 32 lane slots; slot l accumulates, for
// groups g = l, l+32, ... < G and passes p in order,
//     s_l = fmaf(f32(d[t][n][g][p]), ws[n][g] * as[p][t][g], s_l)
// with d the exact int32 dot of the group's 32 codes; the 32 slot sums are
// then reduced by a shfl_down 16/8/4/2/1 tree and rounded to fp16.
//
// Here every d is one v_mfma_i32_16x16x32_i8 (K = 32 = one group), exact in
// int32. The tree pairs slots l and l+16 first, then l and l+8 (of those
// sums), then +4, +2, +1. Five nested two-way loops over the slot bits
// h0 (value 16), h1 (8), h2 (4), h3 (2), h4 (1), innermost h0, visit the
// slots so that each level's pair completes consecutively: every level keeps
// one accumulator per output that takes the first operand of its pair and
// then adds the second, which reproduces the tree's additions exactly.
//
// Tiling: a 256-thread workgroup computes 64 tokens x 64 rows; wave (wm, wn)
// computes 32 x 32 as 2 x 2 sub-tiles of 16 x 16. Per slot the workgroup
// stages the activation scales of its 64 tokens and the weight scales of its
// 64 rows, for all of the slot's groups, in LDS.
#include "common.hpp"

#include <algorithm>

namespace vt {
namespace {

typedef int int4v __attribute__((ext_vector_type(4)));

constexpr int kTile = 64;
constexpr int kMaxSlotGroups = 24;  // groups per slot ceil(G/32) <= 24, i.e. k <= 24576

template <int P>
__global__ __launch_bounds__(256) void a8_gemm(const std::int8_t* __restrict__ acodes,
                                               const float* __restrict__ ascales,
                                               const std::int8_t* __restrict__ wcodes,
                                               const __half* __restrict__ wscales, __half* __restrict__ out,
                                               int tokens, int n, int k, int padded, int groups) {
    // Scales of the current slot's groups (slot + 32*i) for the tile.
    __shared__ float as_lds[P][kMaxSlotGroups][kTile];
    __shared__ float ws_lds[kMaxSlotGroups][kTile];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int q = lane >> 4, r = lane & 15;
    const int t0 = blockIdx.y * kTile, n0 = blockIdx.x * kTile;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const int per_slot = (groups + 31) / 32;

    // Operand rows of this lane (clamped; clamped rows are never stored).
    const std::int8_t* arow[P][2];
    const std::int8_t* brow[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        const std::int64_t t = min(t0 + wm * 32 + a * 16 + r, tokens - 1);
#pragma unroll
        for (int p = 0; p < P; ++p) arow[p][a] = acodes + ((p * count) + t * groups) * 32 + 8 * q;
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const std::int64_t row = min(n0 + wn * 32 + b * 16 + r, n - 1);
        brow[b] = wcodes + row * padded + 8 * q;
    }

    // Level accumulators: lv[0] = slot pair (l, l+16), lv[1] = (+8), ... lv[4] = root.
    float lv[5][16];
    for (int h4 = 0; h4 < 2; ++h4)
        for (int h3 = 0; h3 < 2; ++h3)
            for (int h2 = 0; h2 < 2; ++h2)
                for (int h1 = 0; h1 < 2; ++h1)
                    for (int h0 = 0; h0 < 2; ++h0) {
                        const int slot = h4 + 2 * h3 + 4 * h2 + 8 * h1 + 16 * h0;
                        __syncthreads();
                        for (int e = threadIdx.x; e < per_slot * kTile; e += 256) {
                            const int i = e / kTile, col = e % kTile;
                            const int g = min(slot + 32 * i, groups - 1);
                            const std::int64_t t = min(t0 + col, tokens - 1);
#pragma unroll
                            for (int p = 0; p < P; ++p) as_lds[p][i][col] = ascales[p * count + t * groups + g];
                            const std::int64_t row = min(n0 + col, n - 1);
                            ws_lds[i][col] = __half2float(wscales[row * (padded / 32) + g]);
                        }
                        __syncthreads();

                        float s[16];
#pragma unroll
                        for (int o = 0; o < 16; ++o) s[o] = 0.0f;
                        int i = 0;
                        for (int g = slot; g < groups; g += 32, ++i) {
                            long av[P][2], bv[2];
#pragma unroll
                            for (int a = 0; a < 2; ++a)
#pragma unroll
                                for (int p = 0; p < P; ++p)
                                    av[p][a] = *reinterpret_cast<const long*>(arow[p][a] + g * 32);
#pragma unroll
                            for (int b = 0; b < 2; ++b) bv[b] = *reinterpret_cast<const long*>(brow[b] + g * 32);
                            float ws[2];
#pragma unroll
                            for (int b = 0; b < 2; ++b) ws[b] = ws_lds[i][wn * 32 + b * 16 + r];
#pragma unroll
                            for (int p = 0; p < P; ++p) {
#pragma unroll
                                for (int a = 0; a < 2; ++a) {
                                    const float4 as4 =
                                        *reinterpret_cast<const float4*>(&as_lds[p][i][wm * 32 + a * 16 + 4 * q]);
                                    const float asv[4] = {as4.x, as4.y, as4.z, as4.w};
#pragma unroll
                                    for (int b = 0; b < 2; ++b) {
                                        const int4v zero = {0, 0, 0, 0};
                                        const int4v d =
                                            __builtin_amdgcn_mfma_i32_16x16x32_i8(av[p][a], bv[b], zero, 0, 0, 0);
#pragma unroll
                                        for (int e = 0; e < 4; ++e) {
                                            float& acc = s[(a * 2 + b) * 4 + e];
                                            acc = __fmaf_rn(static_cast<float>(d[e]), __fmul_rn(ws[b], asv[e]), acc);
                                        }
                                    }
                                }
                            }
                        }
                        // Fold the slot into the level accumulators: a level takes the
                        // first member of its pair and adds the second.
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
    require((groups + 31) / 32 <= kMaxSlotGroups, "the A8 GEMM supports k <= 24576");
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const auto* acodes = static_cast<const std::int8_t*>(workspace);
    const auto* ascales = reinterpret_cast<const float*>(acodes + count * 32 * passes);
    const dim3 grid((n + kTile - 1) / kTile, (tokens + kTile - 1) / kTile);
    require(grid.y <= 65535, "token tiles exceed the launch grid");
    if (passes == 1)
        a8_gemm<1><<<grid, 256, 0, stream>>>(acodes, ascales, codes, scales, static_cast<__half*>(out), tokens, n, k,
                                              padded, groups);
    else
        a8_gemm<2><<<grid, 256, 0, stream>>>(acodes, ascales, codes, scales, static_cast<__half*>(out), tokens, n, k,
                                              padded, groups);
}

}  // namespace vt
