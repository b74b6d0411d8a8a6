// W8A8 projection at decode token counts (1..32) on int8 matrix cores, over
// the tiled Q8 planes of the A16 decode route (the "mfma" A8 route below the
// prefill GEMM's tiles).
//
// out[t][n] = fp16( sum_g d[t][n][g] * (ws[n][g] * as[t][g]) )              (one pass)
// out[t][n] = fp16( sum_g (d1 * as1[t][g] + d0 * as0[t][g]) * ws[n][g] )     (two passes)
//
// d is the exact int32 dot of a 32-column group's activation and weight codes
// (q8_dp4a.cuh:47-58): one v_mfma_i32_16x16x32_i8 per group and 16 x 16
// tile, accumulating from zero, so the integer accumulator is the
// reference's. The group terms use the reference's products and FMA but are
// summed in natural group order into one fp32 per output (the reference
// combines 32 lane slots through a shuffle tree), so outputs agree with the
// reference to fp32 association, as the matrix-core A8 prefill GEMM.
//
// The MFMA computes the transposed tile: A is 16 weight rows x 32 codes, B is
// 32 activation codes x 16 tokens, so lane (q, r) of D holds rows 4q .. 4q+3
// of the row block for token r. With that orientation the tiled planes are
// the A fragments as stored (lane 16q + m holds row m's bytes 8q .. 8q+7 of
// groups 2c and 2c+1 of chunk c, 16 bytes), a lane's four weight-row scales
// of a chunk are one 16-byte load from the tiled scales ([block][chunk][row]
// [2 groups]), and its activation scales are the two of its own token
// ([pass][token][group] fp32, as the workspace holds them). B fragments are
// 8 bytes of the token's group codes at [pass][token][group][8q ..].
//
// Launch: W waves over RB row blocks per workgroup, the chunks split evenly
// over the waves, two batches of one chunk in flight per wave (the loads are
// unconditional and the loop's entry and back edge leave the same requests
// outstanding, so each multiply waits only for its own batch); the W partial
// tiles are summed through LDS in wave order, so results are deterministic.
#include "common.hpp"

namespace vt {
namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

template <int RB, int NB, int P>
struct A8Batch {
    uint4 w[RB];              // 16 weight code bytes per block (groups 2c and 2c + 1)
    uint4 ws[RB];             // four rows' scale pairs (fp16)
    uint2 ac[P][NB][2];       // 8 activation code bytes of groups 2c and 2c + 1
    float as[P][NB][2];       // the token's activation scales of the two groups
    bool pair;                // group 2c + 1 exists (false only in the last chunk of an odd group count)
};

template <int W, int RB, int NB, int P>
__global__ __launch_bounds__(W * 64) void a8_tiled_decode(const std::int8_t* __restrict__ acodes,
                                                          const float* __restrict__ ascales,
                                                          const uint4* __restrict__ codes,
                                                          const uint4* __restrict__ scales, __half* __restrict__ out,
                                                          int tokens, int n, int groups, int chunks, int blocks) {
    // chunks: the plane's chunk stride (padded / 64); the wave loop covers only
    // the ceil(groups / 2) chunks that hold a group of the workspace.
    __shared__ float4v partial[W][RB * NB][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int block0 = blockIdx.x * RB;
    const int used = (groups + 1) / 2;
    const int per = (used + W - 1) / W;
    const int c0 = min(wave * per, used), c1 = min(c0 + per, used);
    const int batches = c1 - c0;  // one chunk per batch
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;

    // Activation sources of this lane's token (absent tokens read the last
    // token's codes and feed only outputs that are never stored).
    const std::int8_t* arow[P][NB];
    const float* srow[P][NB];
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
        for (int tb = 0; tb < NB; ++tb) {
            const std::int64_t t = min(16 * tb + r, tokens - 1);
            arow[p][tb] = acodes + (p * count + t * groups) * 32 + 8 * q;
            srow[p][tb] = ascales + p * count + t * groups;
        }
    const uint4* wsrc[RB];
    const uint4* ssrc[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const std::int64_t blk = min(block0 + b, blocks - 1);  // clamped blocks are never stored
        wsrc[b] = codes + blk * chunks * 64 + lane;
        ssrc[b] = scales + blk * chunks * 4 + q;
    }

    // Chunk i of the wave (clamped to its last chunk past the end: re-read, never
    // multiplied). In the last chunk of an odd group count the second group is
    // not the workspace's: its loads re-read the last group and its term is
    // skipped (the weight codes and scales of padded groups are not read into
    // any output, as in the reference, which stops at the last group).
    auto fetch = [&](int i, A8Batch<RB, NB, P>& t) {
        const int ch = min(c0 + i, c1 - 1);
        t.pair = 2 * ch + 1 < groups;
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            t.w[b] = stream_load(wsrc[b] + static_cast<std::int64_t>(ch) * 64);
            t.ws[b] = stream_load(ssrc[b] + static_cast<std::int64_t>(ch) * 4);
        }
        const int ga = min(2 * ch, groups - 1), gb = min(2 * ch + 1, groups - 1);
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int tb = 0; tb < NB; ++tb) {
                t.ac[p][tb][0] = *reinterpret_cast<const uint2*>(arow[p][tb] + ga * 32);
                t.ac[p][tb][1] = *reinterpret_cast<const uint2*>(arow[p][tb] + gb * 32);
                t.as[p][tb][0] = srow[p][tb][ga];
                t.as[p][tb][1] = srow[p][tb][gb];
            }
    };

    float4v y[RB][NB];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int tb = 0; tb < NB; ++tb) y[b][tb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    const int4v zero = {0, 0, 0, 0};

    auto consume = [&](const A8Batch<RB, NB, P>& t) {
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const long wa = static_cast<long>(static_cast<unsigned long>(t.w[b].x) | (static_cast<unsigned long>(t.w[b].y) << 32));
            const long wb = static_cast<long>(static_cast<unsigned long>(t.w[b].z) | (static_cast<unsigned long>(t.w[b].w) << 32));
            // Rows 4q + e: scale pairs (group a, group b) in the 32-bit words of t.ws[b].
            const std::uint32_t pair[4] = {t.ws[b].x, t.ws[b].y, t.ws[b].z, t.ws[b].w};
#pragma unroll
            for (int tb = 0; tb < NB; ++tb) {
                int4v da[P], db[P];
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const long xa = static_cast<long>(static_cast<unsigned long>(t.ac[p][tb][0].x) |
                                                      (static_cast<unsigned long>(t.ac[p][tb][0].y) << 32));
                    const long xb = static_cast<long>(static_cast<unsigned long>(t.ac[p][tb][1].x) |
                                                      (static_cast<unsigned long>(t.ac[p][tb][1].y) << 32));
                    da[p] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wa, xa, zero, 0, 0, 0);
                    db[p] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wb, xb, zero, 0, 0, 0);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float wsa = half_lo(pair[e]), wsb = half_hi(pair[e]);
                    if constexpr (P == 1) {
                        y[b][tb][e] = fmaf(static_cast<float>(da[0][e]), wsa * t.as[0][tb][0], y[b][tb][e]);
                        if (t.pair)
                            y[b][tb][e] = fmaf(static_cast<float>(db[0][e]), wsb * t.as[0][tb][1], y[b][tb][e]);
                    } else {
                        const float ta = fmaf(static_cast<float>(da[1][e]), t.as[1][tb][0],
                                              static_cast<float>(da[0][e]) * t.as[0][tb][0]);
                        const float tbv = fmaf(static_cast<float>(db[1][e]), t.as[1][tb][1],
                                               static_cast<float>(db[0][e]) * t.as[0][tb][1]);
                        y[b][tb][e] = fmaf(ta, wsa, y[b][tb][e]);
                        if (t.pair) y[b][tb][e] = fmaf(tbv, wsb, y[b][tb][e]);
                    }
                }
            }
        }
    };

    if (batches > 0) {
        A8Batch<RB, NB, P> ta, tb2;
        fetch(0, ta);
        fetch(1, tb2);
        int i = 0;
        for (; i + 3 < batches; i += 2) {
            consume(ta);
            __builtin_amdgcn_sched_barrier(0);
            fetch(i + 2, ta);
            __builtin_amdgcn_sched_barrier(0);
            consume(tb2);
            __builtin_amdgcn_sched_barrier(0);
            fetch(i + 3, tb2);
            __builtin_amdgcn_sched_barrier(0);
        }
        consume(ta);
        if (i + 2 < batches) fetch(i + 2, ta);
        if (i + 1 < batches) consume(tb2);
        if (i + 2 < batches) consume(ta);
    }
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int tb = 0; tb < NB; ++tb) partial[wave][b * NB + tb][lane] = y[b][tb];
    __syncthreads();
    for (int p = wave; p < RB * NB; p += W) {
        const int b = p / NB, tb = p % NB;
        float4v sum = partial[0][p][lane];
        for (int w = 1; w < W; ++w) {
            const float4v v = partial[w][p][lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) sum[e] += v[e];
        }
        const int blk = block0 + b, t = 16 * tb + r;
        if (blk >= blocks || t >= tokens) continue;
        __half* o = out + static_cast<std::int64_t>(t) * n + 16 * blk + 4 * q;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (16 * blk + 4 * q + e < n) o[e] = from_f32<__half>(sum[e]);
    }
}

template <int W, int RB, int NB, int P>
void launch_a8_tiled(const std::int8_t* acodes, const float* ascales, const uint4* codes, const uint4* scales,
                     __half* out, int tokens, int n, int groups, int chunks, int blocks, hipStream_t stream) {
    a8_tiled_decode<W, RB, NB, P><<<(blocks + RB - 1) / RB, W * 64, 0, stream>>>(acodes, ascales, codes, scales, out,
                                                                                 tokens, n, groups, chunks, blocks);
}

// Shapes (unsplit K). One token block: 16 waves over two row blocks while that
// grid has at most 256 workgroups (one per CU), else 8 waves over three. Two
// token blocks: 8 waves over two row blocks (the other shapes spill).
template <int NB, int P>
void dispatch_a8_tiled(const std::int8_t* acodes, const float* ascales, const uint4* codes, const uint4* scales,
                       __half* out, int tokens, int n, int groups, int chunks, int blocks, hipStream_t stream) {
    if constexpr (NB == 2)
        launch_a8_tiled<8, 2, NB, P>(acodes, ascales, codes, scales, out, tokens, n, groups, chunks, blocks, stream);
    else if ((blocks + 1) / 2 <= 256)
        launch_a8_tiled<16, 2, NB, P>(acodes, ascales, codes, scales, out, tokens, n, groups, chunks, blocks, stream);
    else
        launch_a8_tiled<8, 3, NB, P>(acodes, ascales, codes, scales, out, tokens, n, groups, chunks, blocks, stream);
}

}  // namespace

std::uint64_t a8_bytes(int tokens, int k, int passes);

void a8_tiled_launch(const void* workspace, std::uint64_t available, const void* codes, const void* scales, void* out,
                     int tokens, int n, int k, int padded, int passes, hipStream_t stream) {
    require(workspace && codes && scales && out, "null A8 operand");
    require(tokens > 0 && tokens <= 32, "the matrix-core A8 decode kernel takes 1..32 tokens");
    require(n > 0 && k > 0 && padded == padded_k(k), "invalid A8 projection geometry");
    require(passes == 1 || passes == 2, "A8 passes must be 1 or 2");
    require(static_cast<std::uint64_t>(tokens) * n < INT32_MAX, "A8 output count exceeds int32");
    require(available >= a8_bytes(tokens, k, passes), "invalid A8 workspace size");
    require(aligned(workspace, 16) && aligned(codes, 16) && aligned(scales, 16) && aligned(out, 2),
            "misaligned A8 operand (workspace and tiled planes need 16 bytes)");
    const int groups = (k + 31) / 32;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const auto* acodes = static_cast<const std::int8_t*>(workspace);
    const auto* ascales = reinterpret_cast<const float*>(acodes + count * 32 * passes);
    const auto* cp = static_cast<const uint4*>(codes);
    const auto* sp = static_cast<const uint4*>(scales);
    auto* op = static_cast<__half*>(out);
    const int chunks = padded / 64, blocks = (n + 15) / 16;
    if (tokens <= 16) {
        if (passes == 1) dispatch_a8_tiled<1, 1>(acodes, ascales, cp, sp, op, tokens, n, groups, chunks, blocks, stream);
        else dispatch_a8_tiled<1, 2>(acodes, ascales, cp, sp, op, tokens, n, groups, chunks, blocks, stream);
    } else {
        if (passes == 1) dispatch_a8_tiled<2, 1>(acodes, ascales, cp, sp, op, tokens, n, groups, chunks, blocks, stream);
        else dispatch_a8_tiled<2, 2>(acodes, ascales, cp, sp, op, tokens, n, groups, chunks, blocks, stream);
    }
}

}  // namespace vt

// Extension: the W8A8 projection of venturi_q8_dp4a_run at 1..32 tokens on
// int8 matrix cores over the tiled Q8 planes (the layout of
// venturi_q8_tiled_run); same A8 workspace; outputs equal the reference's up
// to fp32 association (exact int32 group dots, groups summed in natural order).
extern "C" __attribute__((visibility("default"))) int venturi_q8_a8_tiled_run(const void* workspace,
                                                                             std::uint64_t available,
                                                                             const void* codes, const void* scales,
                                                                             void* out, int tokens, int n, int k,
                                                                             int padded, int passes, void* stream) {
    return vt::guarded([&] {
        vt::a8_tiled_launch(workspace, available, codes, scales, out, tokens, n, k, padded, passes,
                            static_cast<hipStream_t>(stream));
    });
}
