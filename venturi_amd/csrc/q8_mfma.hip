// Q8 A16 projection on fp16 matrix cores (the "mfma" route).
//
// out[t][n] = sum_g scale[n][g] * D[t][n][g],  D = sum_{k in g} x[t][k]*code[n][k]
//
// Each 32-column group's dot D is one v_mfma_f32_16x16x32_f16: int8 codes
// are exact in fp16 and x*code products are exact in fp32, so D carries the
// matrix core's fp32 accumulation; the group scale is applied with one fp32
// FMA per (t, n, g). The association differs from the reference's canonical
// per-column order (blocks.cu:306-321), so outputs agree to fp32 rounding
// rather than bit-for-bit; the order is fixed, so results are deterministic.
//
// Decode kernel (tokens <= 16): one 1024-thread workgroup per 16 weight rows;
// its 16 waves split K. Per 64-column step a lane loads 16 code bytes of one
// row (quarter q of the wave holds bytes [16q, 16q+16) of the two groups) and
// one exchange with lane l^32 gives every quarter 8 bytes of each group. The
// K order inside a group is immaterial to the dot as long as activations use
// the same permutation: quarter q holds group columns off(q)..off(q)+7 with
// off = {0, 16, 8, 24}. The 16 partial tiles are summed through LDS in wave
// order 0..15.
#include "common.hpp"

#include <algorithm>

namespace vt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kDecodeWaves = 16;

// Four int8 codes -> four fp16 values, exactly: with u = c + 128 (c ^ 0x80),
// the fp16 pattern 0x6400 | u is 1024 + u, and subtracting 1152 leaves c.
__device__ __forceinline__ void codes_to_half4(std::uint32_t w, std::uint32_t& lo, std::uint32_t& hi) {
    const std::uint32_t u = w ^ 0x80808080u;
    // v_perm_b32 selector bytes: 0..3 pick from src1 (u), 4..7 from src0 (0x64..)
    lo = __builtin_amdgcn_perm(0x64646464u, u, 0x05010400u);  // [u0, 0x64, u1, 0x64]
    hi = __builtin_amdgcn_perm(0x64646464u, u, 0x05030402u);  // [u2, 0x64, u3, 0x64]
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    const half2v bias = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    half2v a = __builtin_bit_cast(half2v, lo) + bias;
    half2v b = __builtin_bit_cast(half2v, hi) + bias;
    lo = __builtin_bit_cast(std::uint32_t, a);
    hi = __builtin_bit_cast(std::uint32_t, b);
}

__device__ __forceinline__ half8 pack8(std::uint32_t a, std::uint32_t b, std::uint32_t c, std::uint32_t d) {
    typedef std::uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = {a, b, c, d};
    return __builtin_bit_cast(half8, v);
}

template <int STEPS>
struct DecodeStep {
    uint4 w[STEPS];              // 16 code bytes per lane per step
    uint4 xa[STEPS], xb[STEPS];  // activations of groups 2s and 2s+1 (8 halves each)
    std::uint32_t sc[STEPS];     // the row's two group scales
};

// grid.x = ceil(n/16); wave w covers 64-column steps [w*per, min((w+1)*per,
// steps)) of the workgroup's 16 rows, issuing the loads of STEPS steps at once.
template <int STEPS>
__global__ __launch_bounds__(1024) void q8_mfma_decode(const __half* __restrict__ x, const std::int8_t* __restrict__ codes,
                                                       const __half* __restrict__ scales, __half* __restrict__ out,
                                                       int tokens, int n, int k, int padded) {
    __shared__ float4v partial[kDecodeWaves][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int row0 = blockIdx.x * 16;
    const std::int64_t row = min(row0 + r, n - 1);
    const int steps = padded >> 6;
    const int per = (steps + kDecodeWaves - 1) / kDecodeWaves;
    const int s0 = wave * per, s1 = min(s0 + per, steps);
    const int groups = padded >> 5;
    const bool live_token = r < tokens;
    const int off = (q == 0) ? 0 : (q == 1) ? 16 : (q == 2) ? 8 : 24;
    const __half* xrow = x + static_cast<std::int64_t>(min(r, tokens - 1)) * k;
    const std::int8_t* crow = codes + row * padded + 16 * q;
    const __half* srow = scales + row * groups;

    float4v y = {0.0f, 0.0f, 0.0f, 0.0f};
    const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s = s0; s < s1; s += STEPS) {
        DecodeStep<STEPS> d;
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
            const int st = min(s + i, s1 - 1);  // clamped repeats are not accumulated
            const int col = st * 64;
            d.w[i] = *reinterpret_cast<const uint4*>(crow + col);
            d.sc[i] = *reinterpret_cast<const std::uint32_t*>(srow + 2 * st);
            d.xa[i] = *reinterpret_cast<const uint4*>(xrow + min(col + off, k - 8));
            d.xb[i] = *reinterpret_cast<const uint4*>(xrow + min(col + 32 + off, k - 8));
        }
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
            if (s + i >= s1) break;
            const int col = (s + i) * 64;
            // Bring group 2s to every quarter's low half and group 2s+1 to the high half.
            const bool lower = lane < 32;
            const std::uint32_t send0 = lower ? d.w[i].z : d.w[i].x;
            const std::uint32_t send1 = lower ? d.w[i].w : d.w[i].y;
            const std::uint32_t recv0 = __shfl_xor(send0, 32, 64);
            const std::uint32_t recv1 = __shfl_xor(send1, 32, 64);
            const std::uint32_t ga0 = lower ? d.w[i].x : recv0, ga1 = lower ? d.w[i].y : recv1;
            const std::uint32_t gb0 = lower ? recv0 : d.w[i].z, gb1 = lower ? recv1 : d.w[i].w;
            std::uint32_t h0, h1, h2, h3, h4, h5, h6, h7;
            codes_to_half4(ga0, h0, h1);
            codes_to_half4(ga1, h2, h3);
            codes_to_half4(gb0, h4, h5);
            codes_to_half4(gb1, h6, h7);
            const bool live_a = live_token && col + off < k;
            const bool live_b = live_token && col + 32 + off < k;
            const half8 xa = live_a ? __builtin_bit_cast(half8, d.xa[i]) : half8{};
            const half8 xb = live_b ? __builtin_bit_cast(half8, d.xb[i]) : half8{};
            const float4v da = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, pack8(h0, h1, h2, h3), zero, 0, 0, 0);
            const float4v db = __builtin_amdgcn_mfma_f32_16x16x32_f16(xb, pack8(h4, h5, h6, h7), zero, 0, 0, 0);
            // Groups entirely past k have D == 0; their stored scales are never used.
            const float sa = col < k ? half_lo(d.sc[i]) : 0.0f;
            const float sb = col + 32 < k ? half_hi(d.sc[i]) : 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                y[j] = fmaf(da[j], sa, y[j]);
                y[j] = fmaf(db[j], sb, y[j]);
            }
        }
    }
    partial[wave][lane] = y;
    __syncthreads();
    if (wave == 0) {
        float4v sum = partial[0][lane];
        for (int w = 1; w < kDecodeWaves; ++w) {
            const float4v p = partial[w][lane];
#pragma unroll
            for (int j = 0; j < 4; ++j) sum[j] += p[j];
        }
        // D layout: lane holds rows (tokens) 4q..4q+3 of weight row r.
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = 4 * q + j;
            if (t < tokens && row0 + r < n)
                out[static_cast<std::int64_t>(t) * n + row0 + r] = from_f32<__half>(sum[j]);
        }
    }
}

// ---------------------------------------------------------------------------
// Tiled Q8 planes for the matrix-core route (built once when a plan is
// prepared): row block b (16 rows) and 64-column chunk c form 1 KB stored
// [b][c][lane l = 16q + m][16 bytes]; lane (m, q) holds row m's codes of
// columns 64c + 8q .. +8 (group 2c) then 64c + 32 + 8q .. +8 (group 2c + 1),
// exactly the two MFMA B-operand fragments it needs. Scales are [b][c][m][2]
// fp16 (groups 2c, 2c + 1 of row m). A wave streams its chunks of a row block
// as contiguous 1 KB loads. Padding rows/columns hold zero codes and scales.
// Workgroup: RB consecutive row blocks; its 16 waves split the chunks, and each
// wave reuses one activation fragment for all RB row blocks of its chunk. NB
// token blocks of 16 (tokens <= 16 * NB) share every weight fragment.
template <int STEPS, int RB, int NB>
__global__ __launch_bounds__(1024) void q8_tiled_decode(const __half* __restrict__ x, const uint4* __restrict__ codes,
                                                        const std::uint32_t* __restrict__ scales,
                                                        __half* __restrict__ out, int tokens, int n, int k,
                                                        int chunks, int blocks) {
    __shared__ float4v partial[kDecodeWaves][RB * NB][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int block0 = blockIdx.x * RB;
    const int per = (chunks + kDecodeWaves - 1) / kDecodeWaves;
    const int c0 = wave * per, c1 = min(c0 + per, chunks);
    bool live_token[NB];
    const __half* xrow[NB];
#pragma unroll
    for (int tb = 0; tb < NB; ++tb) {
        live_token[tb] = 16 * tb + r < tokens;
        xrow[tb] = x + static_cast<std::int64_t>(min(16 * tb + r, tokens - 1)) * k;
    }
    const uint4* wsrc[RB];
    const std::uint32_t* ssrc[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const int blk = min(block0 + b, blocks - 1);  // clamped blocks are never stored
        wsrc[b] = codes + static_cast<std::int64_t>(blk) * chunks * 64 + lane;
        ssrc[b] = scales + static_cast<std::int64_t>(blk) * chunks * 16 + r;
    }

    float4v y[RB][NB];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int tb = 0; tb < NB; ++tb) y[b][tb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c = c0; c < c1; c += STEPS) {
        uint4 w[STEPS][RB], xa[STEPS][NB], xb[STEPS][NB];
        std::uint32_t sc[STEPS][RB];
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
            const int ch = min(c + i, c1 - 1);  // clamped repeats are not accumulated
            const int col = ch * 64 + 8 * q;
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                w[i][b] = wsrc[b][static_cast<std::int64_t>(ch) * 64];
                sc[i][b] = ssrc[b][static_cast<std::int64_t>(ch) * 16];
            }
#pragma unroll
            for (int tb = 0; tb < NB; ++tb) {
                xa[i][tb] = *reinterpret_cast<const uint4*>(xrow[tb] + min(col, k - 8));
                xb[i][tb] = *reinterpret_cast<const uint4*>(xrow[tb] + min(col + 32, k - 8));
            }
        }
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
            if (c + i >= c1) break;
            const int col = (c + i) * 64 + 8 * q;
            half8 fa[NB], fb[NB];
#pragma unroll
            for (int tb = 0; tb < NB; ++tb) {
                fa[tb] = live_token[tb] && col < k ? __builtin_bit_cast(half8, xa[i][tb]) : half8{};
                fb[tb] = live_token[tb] && col + 32 < k ? __builtin_bit_cast(half8, xb[i][tb]) : half8{};
            }
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                std::uint32_t h0, h1, h2, h3, h4, h5, h6, h7;
                codes_to_half4(w[i][b].x, h0, h1);
                codes_to_half4(w[i][b].y, h2, h3);
                codes_to_half4(w[i][b].z, h4, h5);
                codes_to_half4(w[i][b].w, h6, h7);
                const half8 wa = pack8(h0, h1, h2, h3), wb = pack8(h4, h5, h6, h7);
                const float sa = half_lo(sc[i][b]), sb = half_hi(sc[i][b]);  // padded groups carry scale 0
#pragma unroll
                for (int tb = 0; tb < NB; ++tb) {
                    const float4v da = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[tb], wa, zero, 0, 0, 0);
                    const float4v db = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[tb], wb, zero, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        y[b][tb][j] = fmaf(da[j], sa, y[b][tb][j]);
                        y[b][tb][j] = fmaf(db[j], sb, y[b][tb][j]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int tb = 0; tb < NB; ++tb) partial[wave][b * NB + tb][lane] = y[b][tb];
    __syncthreads();
    // Waves 0..RB*NB-1 each reduce one (row block, token block) in wave order 0..15.
    if (wave < RB * NB) {
        const int b = wave / NB, tb = wave % NB;
        float4v sum = partial[0][wave][lane];
        for (int w = 1; w < kDecodeWaves; ++w) {
            const float4v p = partial[w][wave][lane];
#pragma unroll
            for (int j = 0; j < 4; ++j) sum[j] += p[j];
        }
        // D layout: lane holds rows (tokens) 4q..4q+3 of the token block, weight row r.
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = 16 * tb + 4 * q + j;
            const int row = (block0 + b) * 16 + r;
            if (t < tokens && row < n) out[static_cast<std::int64_t>(t) * n + row] = from_f32<__half>(sum[j]);
        }
    }
}

}  // namespace

void q8_tiled_launch(const void* x, const void* codes, const void* scales, void* out, int tokens, int n, int k,
                     int padded, int dtype, hipStream_t stream) {
    require(x && codes && scales && out, "null Q8 operand");
    require(tokens > 0 && n > 0 && k > 0 && padded == padded_k(k), "invalid Q8 geometry");
    require(static_cast<std::int64_t>(tokens) * n < INT32_MAX, "Q8 output count exceeds int32");
    require(dtype == kF16, "the Q8 MFMA route takes FP16 activations");
    require(k % 8 == 0 && aligned(x, 16), "the Q8 MFMA route needs k % 8 == 0 and 16-byte aligned x");
    require(aligned(codes, 16) && aligned(scales, 4) && aligned(out, 2), "misaligned Q8 operand");
    require(tokens <= 32, "the tiled Q8 MFMA decode kernel takes at most 32 tokens");
    // Row blocks per workgroup: every activation fragment a wave loads feeds
    // one MFMA pair per row block, so more blocks cut the activation traffic
    // through the vector L1, which grows with the token count; fewer blocks
    // keep more workgroups in flight. Two blocks (four steps of 1 KB each in
    // flight per block) below 8 tokens or on matrices of fewer than 1024
    // blocks; four blocks (two steps) otherwise. Both measured on the
    // config-2 shapes.
    const int blocks = (n + 15) / 16;
    const auto* xp = static_cast<const __half*>(x);
    const auto* cp = static_cast<const uint4*>(codes);
    const auto* sp = static_cast<const std::uint32_t*>(scales);
    auto* op = static_cast<__half*>(out);
    if (tokens <= 16 && tokens >= 8 && blocks >= 1024)
        q8_tiled_decode<2, 4, 1><<<(blocks + 3) / 4, 1024, 0, stream>>>(xp, cp, sp, op, tokens, n, k, padded / 64, blocks);
    else if (tokens <= 16)
        q8_tiled_decode<4, 2, 1><<<(blocks + 1) / 2, 1024, 0, stream>>>(xp, cp, sp, op, tokens, n, k, padded / 64, blocks);
    else
        q8_tiled_decode<4, 2, 2><<<(blocks + 1) / 2, 1024, 0, stream>>>(xp, cp, sp, op, tokens, n, k, padded / 64, blocks);
}

void q8_mfma_launch(const void* x, const std::int8_t* codes, const __half* scales, void* out, int tokens, int n,
                    int k, int padded, int dtype, hipStream_t stream) {
    require(x && codes && scales && out, "null Q8 operand");
    require(tokens > 0 && n > 0 && k > 0 && padded == padded_k(k), "invalid Q8 geometry");
    require(static_cast<std::int64_t>(tokens) * n < INT32_MAX, "Q8 output count exceeds int32");
    require(dtype == kF16, "the Q8 MFMA route takes FP16 activations");
    require(k % 8 == 0 && aligned(x, 16), "the Q8 MFMA route needs k % 8 == 0 and 16-byte aligned x");
    require(aligned(codes, 16) && aligned(scales, 4) && aligned(out, 2), "misaligned Q8 operand");
    require(tokens <= 16, "the Q8 MFMA decode kernel takes at most 16 tokens");
    // One workgroup per 16 rows; each wave issues up to 6 steps (6 KB of codes,
    // 12 KB of activations) at once.
    const dim3 grid((n + 15) / 16);
    q8_mfma_decode<6><<<grid, 1024, 0, stream>>>(static_cast<const __half*>(x), codes, scales,
                                                  static_cast<__half*>(out), tokens, n, k, padded);
}

}  // namespace vt

// Extension: the Q8 A16 projection on matrix cores (same arguments as
// venturi_q8_head_run; fp16 activations, tokens <= 16 in this build).
extern "C" __attribute__((visibility("default"))) int venturi_q8_gemm_run(const void* x, const std::int8_t* codes,
                                                                         const __half* scales, void* out, int tokens,
                                                                         int n, int k, int padded, int dtype,
                                                                         void* stream) {
    return vt::guarded([&] {
        vt::q8_mfma_launch(x, codes, scales, out, tokens, n, k, padded, dtype, static_cast<hipStream_t>(stream));
    });
}

// Extension: the matrix-core Q8 A16 projection over tiled planes (row blocks of
// 16 x 64-column chunks, 1 KB each, lane-ordered; scales [block][chunk][row][2]).
extern "C" __attribute__((visibility("default"))) int venturi_q8_tiled_run(const void* x, const void* codes,
                                                                          const void* scales, void* out, int tokens,
                                                                          int n, int k, int padded, int dtype,
                                                                          void* stream) {
    return vt::guarded([&] {
        vt::q8_tiled_launch(x, codes, scales, out, tokens, n, k, padded, dtype, static_cast<hipStream_t>(stream));
    });
}
