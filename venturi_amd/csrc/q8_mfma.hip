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
// fp16 (groups 2c, 2c + 1 of row m). Padding rows hold zero codes and scales.
//
// Workgroup: W waves over RB consecutive row blocks. Wave w owns the chunk
// range [w*per, (w+1)*per) of every one of them and streams it in batches of
// STEPS chunks with a two-deep ping-pong: the codes, scales and activation
// fragments of batch i+1 are in flight while batch i is multiplied. Each
// activation fragment feeds one MFMA pair per row block; NB token blocks of
// 16 (tokens <= 16 * NB) share every weight fragment. Only lanes whose token
// row exists load activations (the others hold zeros), so small token counts
// cost no activation traffic beyond their rows. The W partial tiles are summed
// through LDS in wave order 0..W-1, so results are deterministic.
// Writes one projection output: row slot r of 16-row block blk for token t.
// Plain: out[t][16 blk + r], n rows. SwiGLU (paired planes, n = 2 * inter):
// slots 0..7 of block blk are gate rows 8 blk .. 8 blk + 7 and slots 8..15
// the matching up rows; every lane fetches its partner slot's sum (lane ^ 8)
// and lanes of gate slots write out[t][8 blk + r] = swiglu(gate, up), with
// gate and up rounded to fp16 first as the projection would store them. All
// lanes of the wave must call it together.
template <bool SWIGLU>
__device__ __forceinline__ void store_tile_value(__half* __restrict__ out, float v, int t, int blk, int r, int tokens,
                                                 int n) {
    if constexpr (SWIGLU) {
        const float other = __shfl_xor(v, 8, 64);
        const int inter = n / 2, col = 8 * blk + r;
        if (r < 8 && t < tokens && col < inter) {
            const float g = __half2float(from_f32<__half>(v)), u = __half2float(from_f32<__half>(other));
            out[static_cast<std::int64_t>(t) * inter + col] = from_f32<__half>(swiglu_value(g, u));
        }
    } else {
        const int row = 16 * blk + r;
        if (t < tokens && row < n) out[static_cast<std::int64_t>(t) * n + row] = from_f32<__half>(v);
    }
}

// Slot state between the two K halves of a split projection: both fp32 halves
// hold a signalling-NaN pattern, which no arithmetic result takes (NaN results
// are quiet), so a stored partial sum never reads as empty.
constexpr unsigned long long kSlotEmpty = 0x7f8000017f800001ull;

// Writes rows r and r + 8 of 16-row block blk for token t (plain), or the
// SwiGLU of gate slot r and up slot r + 8 (paired planes).
template <bool SWIGLU>
__device__ __forceinline__ void store_row_pair(__half* __restrict__ out, float lo, float hi, int t, int blk, int r,
                                               int n) {
    if constexpr (SWIGLU) {
        const int inter = n / 2, col = 8 * blk + r;
        if (col < inter) {
            const float g = __half2float(from_f32<__half>(lo)), u = __half2float(from_f32<__half>(hi));
            out[static_cast<std::int64_t>(t) * inter + col] = from_f32<__half>(swiglu_value(g, u));
        }
    } else {
        const int row = 16 * blk + r;
        __half* o = out + static_cast<std::int64_t>(t) * n;
        if (row < n) o[row] = from_f32<__half>(lo);
        if (row + 8 < n) o[row + 8] = from_f32<__half>(hi);
    }
}

// Final sums of one 16x16 output tile in the MFMA D layout: lane (q, r) holds
// tokens t0 + 4q + j (j = 0..3) of row slot r of block blk. All lanes of the
// wave call it together.
//
// KS == 1: the tile covers all of K and is stored. KS == 2: the tile is one of
// two K halves computed by different workgroups. Lanes r < 8 exchange the pair
// (own sum, sum of slot r + 8) with the 64-bit slot of (t, blk, r): the first
// half to arrive finds kSlotEmpty and leaves its pair; the second takes the
// other pair, adds it, resets the slot and stores. The sum of two fp32 terms
// does not depend on their order, so the output is the same whichever half
// arrives first. Only the slot itself is shared, so the exchange needs no
// fence, and no wave waits for another.
template <int KS, bool SWIGLU>
__device__ __forceinline__ void finish_tile(__half* __restrict__ out, unsigned long long* __restrict__ slots,
                                            const float4v& sum, int t0, int q, int blk, int r, int tokens, int n,
                                            int blocks) {
    if constexpr (KS == 1) {
#pragma unroll
        for (int j = 0; j < 4; ++j) store_tile_value<SWIGLU>(out, sum[j], t0 + 4 * q + j, blk, r, tokens, n);
    } else {
        static_assert(KS == 2, "K is split in two at most");
        // All four exchanges of a lane are issued before any result is used, so
        // the wave waits for one atomic round trip instead of four in sequence.
        float partner[4];
        unsigned long long old[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) partner[j] = __shfl_xor(sum[j], 8, 64);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = t0 + 4 * q + j;
            old[j] = kSlotEmpty;
            if (r < 8 && t < tokens) {
                unsigned long long* slot = slots + (static_cast<std::int64_t>(t) * blocks + blk) * 8 + r;
                const unsigned long long packed =
                    (static_cast<unsigned long long>(__float_as_uint(partner[j])) << 32) | __float_as_uint(sum[j]);
                old[j] = __hip_atomic_exchange(slot, packed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = t0 + 4 * q + j;
            if (r < 8 && t < tokens && old[j] != kSlotEmpty) {
                unsigned long long* slot = slots + (static_cast<std::int64_t>(t) * blocks + blk) * 8 + r;
                __hip_atomic_store(slot, kSlotEmpty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float lo = sum[j] + __uint_as_float(static_cast<std::uint32_t>(old[j]));
                const float hi = partner[j] + __uint_as_float(static_cast<std::uint32_t>(old[j] >> 32));
                store_row_pair<SWIGLU>(out, lo, hi, t, blk, r, n);
            }
        }
    }
}

template <int RB, int NB, int STEPS>
struct TiledBatch {
    uint4 w[STEPS][RB];
    std::uint32_t sc[STEPS][RB];
    uint4 xa[STEPS][NB], xb[STEPS][NB];
};

// K range of a workgroup: with KS == 2 consecutive workgroups 2g and 2g + 1
// take chunks [0, ceil(chunks/2)) and the rest of row-block group g. The W
// waves split that range evenly.
struct ChunkRange {
    int k0, k1;  // the workgroup's chunks
    int c0, c1;  // this wave's chunks
};

template <int W, int KS>
__device__ __forceinline__ ChunkRange chunk_range(int chunks, int wave) {
    const int ks = KS == 1 ? 0 : static_cast<int>(blockIdx.x % KS);
    const int kper = (chunks + KS - 1) / KS;
    ChunkRange c;
    c.k0 = min(ks * kper, chunks);
    c.k1 = min(c.k0 + kper, chunks);
    const int per = (c.k1 - c.k0 + W - 1) / W;
    c.c0 = min(c.k0 + wave * per, c.k1);
    c.c1 = min(c.c0 + per, c.k1);
    return c;
}

template <int W, int RB, int NB, int STEPS, int KS, bool SWIGLU>
__global__ __launch_bounds__(W * 64) void q8_tiled_decode(const __half* __restrict__ x, const uint4* __restrict__ codes,
                                                          const std::uint32_t* __restrict__ scales,
                                                          __half* __restrict__ out, unsigned long long* __restrict__ slots,
                                                          int tokens, int n, int k, int chunks, int blocks) {
    __shared__ float4v partial[W][RB * NB][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int block0 = static_cast<int>(blockIdx.x / KS) * RB;
    const ChunkRange range = chunk_range<W, KS>(chunks, wave);
    const int c0 = range.c0, c1 = range.c1;
    const int batches = (c1 - c0 + STEPS - 1) / STEPS;
    bool live[NB];
    const __half* xrow[NB];
#pragma unroll
    for (int tb = 0; tb < NB; ++tb) {
        live[tb] = 16 * tb + r < tokens;
        xrow[tb] = x + static_cast<std::int64_t>(min(16 * tb + r, tokens - 1)) * k + 8 * q;
    }
    const uint4* wsrc[RB];
    const std::uint32_t* ssrc[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const int blk = min(block0 + b, blocks - 1);  // clamped blocks are never stored
        wsrc[b] = codes + static_cast<std::int64_t>(blk) * chunks * 64 + lane;
        ssrc[b] = scales + static_cast<std::int64_t>(blk) * chunks * 16 + r;
    }

    // Batch i covers chunks c0 + i*STEPS .. ; chunks past c1 are clamped to
    // c1 - 1 when loaded and skipped when multiplied.
    auto fetch = [&](int i, TiledBatch<RB, NB, STEPS>& t) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
            const int ch = min(c0 + i * STEPS + s, c1 - 1);
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                t.w[s][b] = stream_load(wsrc[b] + static_cast<std::int64_t>(ch) * 64);
                t.sc[s][b] = stream_load(ssrc[b] + static_cast<std::int64_t>(ch) * 16);
            }
        }
        // Activation fragments, branch-free so that the wait counts stay exact:
        // read at clamped in-bounds columns (lanes of absent tokens read the last
        // token's row and feed only output rows never stored); the multiply
        // zeroes columns at or past k.
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
            const int col = min(c0 + i * STEPS + s, c1 - 1) * 64;
#pragma unroll
            for (int tb = 0; tb < NB; ++tb) {
                t.xa[s][tb] = *reinterpret_cast<const uint4*>(xrow[tb] + min(col, k - 8 - 8 * q));
                t.xb[s][tb] = *reinterpret_cast<const uint4*>(xrow[tb] + min(col + 32, k - 8 - 8 * q));
            }
        }
    };

    float4v y[RB][NB];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int tb = 0; tb < NB; ++tb) y[b][tb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};

    auto consume = [&](int i, const TiledBatch<RB, NB, STEPS>& t) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
            const int ch = c0 + i * STEPS + s;
            if (ch >= c1) break;
            const int col = ch * 64 + 8 * q;
            const bool inside = ch * 64 + 64 <= k;  // wave-uniform
            half8 fa[NB], fb[NB];
#pragma unroll
            for (int tb = 0; tb < NB; ++tb) {
                // In the chunk that crosses k, columns at or past k are zero (the
                // clamped load read other columns).
                fa[tb] = inside || col < k ? __builtin_bit_cast(half8, t.xa[s][tb]) : half8{};
                fb[tb] = inside || col + 32 < k ? __builtin_bit_cast(half8, t.xb[s][tb]) : half8{};
            }
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                std::uint32_t h0, h1, h2, h3, h4, h5, h6, h7;
                codes_to_half4(t.w[s][b].x, h0, h1);
                codes_to_half4(t.w[s][b].y, h2, h3);
                codes_to_half4(t.w[s][b].z, h4, h5);
                codes_to_half4(t.w[s][b].w, h6, h7);
                const half8 wa = pack8(h0, h1, h2, h3), wb = pack8(h4, h5, h6, h7);
                const float sa = half_lo(t.sc[s][b]), sb = half_hi(t.sc[s][b]);  // padded groups carry scale 0
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
    };

    // Two batches in flight. Batches 0 and 1 are requested up front (with one
    // batch, the second request re-reads its last chunk and is never used), and
    // in the steady state each multiply is followed by the request that reuses
    // its registers, so every multiply waits only for its own batch while the
    // other is in flight. The loop's loads are unconditional and its entry and
    // back edge leave the same requests outstanding: a conditional request, or
    // a loop entered with fewer requests in flight, makes the compiler's wait
    // counts assume the worst and drain the prefetch. The scheduling barriers
    // keep the compiler from sinking a request below the next multiply.
    if (batches > 0) {
        TiledBatch<RB, NB, STEPS> ta, tb2;
        fetch(0, ta);
        fetch(1, tb2);
        int i = 0;
        for (; i + 3 < batches; i += 2) {
            consume(i, ta);
            __builtin_amdgcn_sched_barrier(0);
            fetch(i + 2, ta);
            __builtin_amdgcn_sched_barrier(0);
            consume(i + 1, tb2);
            __builtin_amdgcn_sched_barrier(0);
            fetch(i + 3, tb2);
            __builtin_amdgcn_sched_barrier(0);
        }
        // One to three batches left: i, i + 1, i + 2.
        consume(i, ta);
        if (i + 2 < batches) fetch(i + 2, ta);
        if (i + 1 < batches) consume(i + 1, tb2);
        if (i + 2 < batches) consume(i + 2, ta);
    }
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int tb = 0; tb < NB; ++tb) partial[wave][b * NB + tb][lane] = y[b][tb];
    __syncthreads();
    // Waves 0..RB*NB-1 each reduce one (row block, token block) in wave order.
    for (int p = wave; p < RB * NB; p += W) {
        const int b = p / NB, tb = p % NB;
        float4v sum = partial[0][p][lane];
        for (int w = 1; w < W; ++w) {
            const float4v v = partial[w][p][lane];
#pragma unroll
            for (int j = 0; j < 4; ++j) sum[j] += v[j];
        }
        // D layout: lane holds rows (tokens) 4q..4q+3 of the token block, weight row r.
        if (block0 + b < blocks) finish_tile<KS, SWIGLU>(out, slots, sum, 16 * tb, q, block0 + b, r, tokens, n, blocks);
    }
}

// The same projection with the activations staged in LDS once per workgroup
// (used when tokens x padded columns fit). Rows 0..tokens-1 hold x with zeros
// from column k up to the padded width, so no fragment needs masking; lanes of
// token rows that do not exist read a 128-byte zero block. Row t's 16-byte
// units are stored XOR-swizzled by (t & 7) inside each 128-byte span, so the
// 16 token rows of one fragment read land in distinct banks. After the main
// loop the LDS holds the per-wave partial tiles instead. TMAX bounds the
// token count (1, 4 or 16): with one token only the first accumulator of each
// lane is live, so the group scaling costs one FMA per group instead of four.
template <int RB, int STEPS>
struct LdsBatch {
    uint4 w[STEPS][RB];
    std::uint32_t sc[STEPS][RB];
};

__host__ __device__ inline std::size_t lds_x_bytes(int tokens, int chunks) {
    return static_cast<std::size_t>(tokens) * chunks * 128 + (tokens < 16 ? 128 : 0);
}

template <int W, int RB, int STEPS, int TMAX, int KS, bool SWIGLU>
__global__ __launch_bounds__(W * 64) void q8_tiled_lds(const __half* __restrict__ x, const uint4* __restrict__ codes,
                                                       const std::uint32_t* __restrict__ scales,
                                                       __half* __restrict__ out, unsigned long long* __restrict__ slots,
                                                       int tokens, int n, int k, int chunks, int blocks) {
    extern __shared__ uint4 lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int block0 = static_cast<int>(blockIdx.x / KS) * RB;
    const ChunkRange range = chunk_range<W, KS>(chunks, wave);
    const int c0 = range.c0, c1 = range.c1;
    const int batches = (c1 - c0 + STEPS - 1) / STEPS;
    const uint4* wsrc[RB];
    const std::uint32_t* ssrc[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const int blk = min(block0 + b, blocks - 1);  // clamped blocks are never stored
        wsrc[b] = codes + static_cast<std::int64_t>(blk) * chunks * 64 + lane;
        ssrc[b] = scales + static_cast<std::int64_t>(blk) * chunks * 16 + r;
    }
    auto fetch = [&](int i, LdsBatch<RB, STEPS>& t) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
            const int ch = min(c0 + i * STEPS + s, c1 - 1);
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                t.w[s][b] = stream_load(wsrc[b] + static_cast<std::int64_t>(ch) * 64);
                t.sc[s][b] = stream_load(ssrc[b] + static_cast<std::int64_t>(ch) * 16);
            }
        }
    };
    // The first two weight batches are in flight while the activations are
    // staged (with one batch, the second request re-reads its last chunk).
    LdsBatch<RB, STEPS> ta, tb2;
    if (batches > 0) {
        fetch(0, ta);
        fetch(1, tb2);
    }

    // Staged row t holds columns [64 k0, 64 k1) of the workgroup's K range.
    const int units = (range.k1 - range.k0) * 8;  // 16-byte units per staged row
    for (int i = threadIdx.x; i < tokens * units; i += W * 64) {
        const int t = i / units, u = i - t * units;
        const int col = 64 * range.k0 + 8 * u;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (col < k) v = *reinterpret_cast<const uint4*>(x + static_cast<std::int64_t>(t) * k + col);
        lds[t * units + (u ^ (t & 7))] = v;
    }
    if (tokens < 16 && threadIdx.x < 8) lds[tokens * units + threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();

    // Fragment addresses (in 16-byte units): chunk ch, group half g (0 or 1)
    // of lane (r, q) is unit ch*8 + 4g + q of row r, swizzled.
    const bool live = r < tokens;
    const int rowbase = live ? r * units : tokens * units;
    const int swz = live ? (r & 7) : 0;
    const int step = live ? 8 : 0;

    float4v y[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) y[b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
    auto consume = [&](int i, const LdsBatch<RB, STEPS>& t) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
            const int ch = c0 + i * STEPS + s;
            if (ch >= c1) break;
            const int base = rowbase + (ch - range.k0) * step;
            const half8 fa = __builtin_bit_cast(half8, lds[base + ((q) ^ swz)]);
            const half8 fb = __builtin_bit_cast(half8, lds[base + ((4 + q) ^ swz)]);
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                std::uint32_t h0, h1, h2, h3, h4, h5, h6, h7;
                codes_to_half4(t.w[s][b].x, h0, h1);
                codes_to_half4(t.w[s][b].y, h2, h3);
                codes_to_half4(t.w[s][b].z, h4, h5);
                codes_to_half4(t.w[s][b].w, h6, h7);
                const half8 wa = pack8(h0, h1, h2, h3), wb = pack8(h4, h5, h6, h7);
                const float sa = half_lo(t.sc[s][b]), sb = half_hi(t.sc[s][b]);  // padded groups carry scale 0
                const float4v da = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa, wa, zero, 0, 0, 0);
                const float4v db = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb, wb, zero, 0, 0, 0);
                constexpr int live_acc = TMAX == 1 ? 1 : 4;
#pragma unroll
                for (int j = 0; j < live_acc; ++j) {
                    y[b][j] = fmaf(da[j], sa, y[b][j]);
                    y[b][j] = fmaf(db[j], sb, y[b][j]);
                }
            }
        }
    };
    // Two batches in flight, pipelined as in q8_tiled_decode; batches 0 and 1
    // were requested before the staging.
    if (batches > 0) {
        int i = 0;
        for (; i + 3 < batches; i += 2) {
            consume(i, ta);
            __builtin_amdgcn_sched_barrier(0);
            fetch(i + 2, ta);
            __builtin_amdgcn_sched_barrier(0);
            consume(i + 1, tb2);
            __builtin_amdgcn_sched_barrier(0);
            fetch(i + 3, tb2);
            __builtin_amdgcn_sched_barrier(0);
        }
        consume(i, ta);
        if (i + 2 < batches) fetch(i + 2, ta);
        if (i + 1 < batches) consume(i + 1, tb2);
        if (i + 2 < batches) consume(i + 2, ta);
    }
    __syncthreads();  // every wave is done with the staged activations
    float4v* partial = reinterpret_cast<float4v*>(lds);  // [W][RB][64]
#pragma unroll
    for (int b = 0; b < RB; ++b) partial[(wave * RB + b) * 64 + lane] = y[b];
    __syncthreads();
    for (int b = wave; b < RB; b += W) {
        float4v sum = partial[b * 64 + lane];
        for (int w = 1; w < W; ++w) {
            const float4v v = partial[(w * RB + b) * 64 + lane];
#pragma unroll
            for (int j = 0; j < 4; ++j) sum[j] += v[j];
        }
        if (block0 + b < blocks) finish_tile<KS, SWIGLU>(out, slots, sum, 0, q, block0 + b, r, tokens, n, blocks);
    }
}

template <int W, int RB, int STEPS, int TMAX, int KS, bool SWIGLU>
void launch_tiled_lds(const __half* x, const uint4* codes, const std::uint32_t* scales, __half* out,
                      unsigned long long* slots, int tokens, int n, int k, int chunks, int blocks, hipStream_t stream) {
    const int kper = (chunks + KS - 1) / KS;
    const std::size_t lds = std::max(lds_x_bytes(tokens, kper), static_cast<std::size_t>(W) * RB * 1024);
    require(lds <= 160 * 1024, "staged activations exceed LDS");
    require(KS == 1 || slots, "a split projection needs its slot buffer");
    static const hipError_t raised =
        hipFuncSetAttribute(reinterpret_cast<const void*>(q8_tiled_lds<W, RB, STEPS, TMAX, KS, SWIGLU>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    check(raised);
    q8_tiled_lds<W, RB, STEPS, TMAX, KS, SWIGLU><<<(blocks + RB - 1) / RB * KS, W * 64, lds, stream>>>(
        x, codes, scales, out, slots, tokens, n, k, chunks, blocks);
}

template <int W, int RB, int NB, int STEPS, int KS, bool SWIGLU>
void launch_tiled(const __half* x, const uint4* codes, const std::uint32_t* scales, __half* out,
                  unsigned long long* slots, int tokens, int n, int k, int chunks, int blocks, hipStream_t stream) {
    require(KS == 1 || slots, "a split projection needs its slot buffer");
    q8_tiled_decode<W, RB, NB, STEPS, KS, SWIGLU><<<(blocks + RB - 1) / RB * KS, W * 64, 0, stream>>>(
        x, codes, scales, out, slots, tokens, n, k, chunks, blocks);
}

// Launch shapes, measured on the config-2 matrices (QKV 7168x5120, o_proj
// 5120x6144, gate+up 34816x5120, down 5120x17408) at 1-32 tokens. A workgroup
// streams at most about 28 GB/s, so the grid should give every CU one
// workgroup of equal work: with fewer than 1024 row blocks, two workgroups on
// one CU finish last and set the time.
//
// One token: activations staged in LDS; 16 waves over one row block (four
// chunks per batch) up to 256 blocks, over two row blocks below 1024 blocks,
// else 8 waves over three (one chunk per batch: with two, the two batches in
// flight hold 12 KB per wave and gate+up at one token measured 32.0 against
// 29.9 us). Long rows (at least 128 chunks) of 257-384 blocks split K instead:
// 8 waves over three blocks and half the chunks, the halves exchanged through
// slots, so 2 * ceil(blocks / 3) workgroups (down, 320 blocks x 272 chunks:
// 214 instead of 160; 19.9 -> 18.7 us). More tokens: register fragments, 8
// waves, one batch of chunks in flight behind the current one, and the
// (row blocks, K halves) shape of the candidates below whose grid is largest
// without passing 256 workgroups; ties go to the unsplit shape up to 16 tokens
// and to more row blocks above (two token blocks load twice the activation
// fragments per weight byte). When none fits, three blocks unsplit.
struct TiledShape {
    bool lds;
    int rb, ks;
};

// Chunk count that admits every split (slot buffers are sized with it, as
// the workspace query does not take K).
constexpr int kAnyChunks = 1 << 30;

TiledShape tiled_shape(int tokens, int blocks, int chunks) {
    // One token: up to 256 row blocks take one block per workgroup (every wave
    // issuing four chunks per batch, two where a wave has at most four),
    // which fills the chip where two blocks per workgroup would leave half of
    // it idle (config 1: 7.3 -> 6.2 us; two-chunk batches 6.3 -> 5.5 us).
    if (tokens == 1) {
        if (blocks <= 256) return TiledShape{true, 1, 1};
        if (blocks < 1024)
            return (blocks + 2) / 3 * 2 <= 256 && chunks >= 128 ? TiledShape{true, 3, 2} : TiledShape{true, 2, 1};
        return TiledShape{true, 3, 1};
    }
    const TiledShape candidates[] = {{false, 2, 1}, {false, 3, 1}, {false, 3, 2}, {false, 4, 2}};
    TiledShape best{false, 3, 1};
    long best_grid = 0;
    for (const TiledShape& c : candidates) {
        const long grid = static_cast<long>((blocks + c.rb - 1) / c.rb) * c.ks;
        if (grid > 256) continue;
        const bool tie_wins = tokens <= 16 ? c.ks < best.ks : c.rb > best.rb;
        if (grid > best_grid || (grid == best_grid && tie_wins)) {
            best = c;
            best_grid = grid;
        }
    }
    return best;
}

std::size_t tiled_slot_bytes(int tokens, int blocks) {
    return tiled_shape(tokens, blocks, kAnyChunks).ks > 1 ? static_cast<std::size_t>(tokens) * blocks * 8 * sizeof(unsigned long long)
                                             : 0;
}

template <int NB, bool SWIGLU>
void launch_tiled_shape(const TiledShape& sh, const __half* xp, const uint4* cp, const std::uint32_t* sp, __half* op,
                        unsigned long long* slots, int tokens, int n, int k, int chunks, int blocks,
                        hipStream_t stream) {
    // Two token blocks with three row blocks need about 154 VGPRs, so one
    // 8-wave workgroup fits a CU (8 waves) where three 4-wave ones do (12
    // waves): grids past 512 workgroups take the 4-wave shape (config-5 gate+up
    // at 32 tokens, 726 workgroups: model step 7.40 -> 7.25 ms). With one
    // token block the 8-wave shape stays faster.
    if (sh.rb == 2 && sh.ks == 1)
        launch_tiled<8, 2, NB, 1, 1, SWIGLU>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else if (NB == 2 && sh.rb == 3 && sh.ks == 1 && (blocks + 2) / 3 > 512)
        launch_tiled<4, 3, NB, 1, 1, SWIGLU>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else if (sh.rb == 3 && sh.ks == 1)
        launch_tiled<8, 3, NB, 1, 1, SWIGLU>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else if (sh.rb == 3 && sh.ks == 2)
        launch_tiled<8, 3, NB, 1, 2, SWIGLU>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else
        launch_tiled<8, 4, NB, 1, 2, SWIGLU>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
}

template <bool SWIGLU>
void tiled_dispatch(const __half* xp, const uint4* cp, const std::uint32_t* sp, __half* op, unsigned long long* slots,
                    int tokens, int n, int k, int chunks, int blocks, hipStream_t stream) {
    const TiledShape sh = tiled_shape(tokens, blocks, chunks);
    if (sh.lds && sh.rb == 1 && chunks <= 64)  // at most four chunks a wave: two batches of two (config 1: 6.3 -> 5.5 us)
        launch_tiled_lds<16, 1, 2, 1, 1, SWIGLU>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else if (sh.lds && sh.rb == 1)
        launch_tiled_lds<16, 1, 4, 1, 1, SWIGLU>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else if (sh.lds && sh.rb == 2)
        launch_tiled_lds<16, 2, 1, 1, 1, SWIGLU>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else if (sh.lds && sh.ks == 2)
        launch_tiled_lds<8, 3, 1, 1, 2, SWIGLU>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else if (sh.lds)
        launch_tiled_lds<8, 3, 1, 1, 1, SWIGLU>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else if (tokens <= 16)
        launch_tiled_shape<1, SWIGLU>(sh, xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else
        launch_tiled_shape<2, SWIGLU>(sh, xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
}

__global__ void fill_slots(unsigned long long* __restrict__ slots, std::size_t count) {
    for (std::size_t i = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; i < count;
         i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
        slots[i] = kSlotEmpty;
}

}  // namespace

int tiled_blocks(int n, bool swiglu) { return swiglu ? (n / 2 + 7) / 8 : (n + 15) / 16; }

std::size_t q8_tiled_workspace_bytes(int tokens, int n, bool swiglu) {
    require(tokens > 0 && tokens <= 32 && n > 0, "invalid Q8 tiled geometry (1..32 tokens, n > 0)");
    require(!swiglu || n % 2 == 0, "the fused SwiGLU projection needs an even row count (gate rows, then up rows)");
    return tiled_slot_bytes(tokens, tiled_blocks(n, swiglu));
}

void q8_tiled_workspace_init(void* workspace, std::size_t bytes, hipStream_t stream) {
    require(bytes % 8 == 0 && (bytes == 0 || (workspace && aligned(workspace, 8))),
            "the Q8 tiled workspace is whole, 8-byte aligned 64-bit words");
    const std::size_t count = bytes / 8;
    if (count == 0) return;
    const int grid = static_cast<int>(std::min<std::size_t>((count + 255) / 256, 1024));
    fill_slots<<<grid, 256, 0, stream>>>(static_cast<unsigned long long*>(workspace), count);
}

void q8_tiled_launch(const void* x, const void* codes, const void* scales, void* out, int tokens, int n, int k,
                     int padded, int dtype, bool swiglu, void* workspace, std::size_t workspace_bytes,
                     hipStream_t stream) {
    require(x && codes && scales && out, "null Q8 operand");
    require(tokens > 0 && n > 0 && k > 0 && padded == padded_k(k), "invalid Q8 geometry");
    require(static_cast<std::int64_t>(tokens) * n < INT32_MAX, "Q8 output count exceeds int32");
    require(dtype == kF16, "the Q8 MFMA route takes FP16 activations");
    require(k % 8 == 0 && aligned(x, 16), "the Q8 MFMA route needs k % 8 == 0 and 16-byte aligned x");
    require(aligned(codes, 16) && aligned(scales, 4) && aligned(out, 2), "misaligned Q8 operand");
    require(tokens <= 32, "the tiled Q8 MFMA decode kernel takes at most 32 tokens");
    require(!swiglu || n % 2 == 0, "the fused SwiGLU projection needs an even row count (gate rows, then up rows)");
    // Paired planes hold 8 gate and 8 up rows per 16-row block.
    const int blocks = tiled_blocks(n, swiglu);
    const std::size_t need = tiled_slot_bytes(tokens, blocks);
    require(need == 0 || (workspace && aligned(workspace, 8) && workspace_bytes >= need),
            "the Q8 tiled projection needs its initialised workspace (venturi_q8_tiled_workspace_bytes)");
    auto* slots = need ? static_cast<unsigned long long*>(workspace) : nullptr;
    const int chunks = padded / 64;
    const auto* xp = static_cast<const __half*>(x);
    const auto* cp = static_cast<const uint4*>(codes);
    const auto* sp = static_cast<const std::uint32_t*>(scales);
    auto* op = static_cast<__half*>(out);
    if (swiglu) tiled_dispatch<true>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    else tiled_dispatch<false>(xp, cp, sp, op, slots, tokens, n, k, chunks, blocks, stream);
    const hipError_t launched = hipGetLastError();
    if (launched != hipSuccess) {
        // A refused launch never ran, so the slots are still idle; refill them
        // anyway (best effort) so that a caller never has to reason about it.
        if (slots) q8_tiled_workspace_init(slots, need, stream);
        check(launched);
    }
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

// Extension: workspace of the tiled projections for (tokens, n): the exchange
// slots of projections whose K is split over two workgroups, or 0 when the
// launch for this shape does not split. Returns 0 with a message on invalid
// arguments.
extern "C" __attribute__((visibility("default"))) std::size_t venturi_q8_tiled_workspace_bytes(int tokens, int n,
                                                                                              int swiglu) {
    std::size_t bytes = 0;
    vt::host_guarded([&] { bytes = vt::q8_tiled_workspace_bytes(tokens, n, swiglu != 0); });
    return bytes;
}

// Extension: puts a tiled-projection workspace in its idle state (a fill
// kernel on `stream`, no memset node). Every projection call leaves it idle.
extern "C" __attribute__((visibility("default"))) int venturi_q8_tiled_workspace_init(void* workspace,
                                                                                     std::size_t bytes,
                                                                                     void* stream) {
    return vt::guarded([&] { vt::q8_tiled_workspace_init(workspace, bytes, static_cast<hipStream_t>(stream)); });
}

// Extension: the matrix-core Q8 A16 projection over tiled planes (row blocks of
// 16 x 64-column chunks, 1 KB each, lane-ordered; scales [block][chunk][row][2]).
extern "C" __attribute__((visibility("default"))) int venturi_q8_tiled_run(const void* x, const void* codes,
                                                                          const void* scales, void* out, int tokens,
                                                                          int n, int k, int padded, int dtype,
                                                                          void* workspace, std::size_t workspace_bytes,
                                                                          void* stream) {
    return vt::guarded([&] {
        vt::q8_tiled_launch(x, codes, scales, out, tokens, n, k, padded, dtype, false, workspace, workspace_bytes,
                            static_cast<hipStream_t>(stream));
    });
}

// Extension: the fused gate+up projection with SwiGLU over paired tiled planes
// (16-row block b = gate rows 8b..8b+7, then up rows inter+8b..inter+8b+7):
// out[t][j] = fp16(swiglu(fp16(gate[t][j]), fp16(up[t][j]))), out [tokens][n/2],
// the bytes of the projection followed by venturi_silu_mul_run.
extern "C" __attribute__((visibility("default"))) int venturi_q8_tiled_swiglu_run(const void* x, const void* codes,
                                                                                 const void* scales, void* out,
                                                                                 int tokens, int n, int k, int padded,
                                                                                 int dtype, void* workspace,
                                                                                 std::size_t workspace_bytes,
                                                                                 void* stream) {
    return vt::guarded([&] {
        vt::q8_tiled_launch(x, codes, scales, out, tokens, n, k, padded, dtype, true, workspace, workspace_bytes,
                            static_cast<hipStream_t>(stream));
    });
}
