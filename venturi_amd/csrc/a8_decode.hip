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
// [2 groups]), and its activation scales are the two of its own token. B
// fragments are 8 bytes of the token's group codes at [group][8q ..].
//
// Three forms share that arithmetic:
// * a8_tiled_decode reads a filled A8 workspace ([pass][token][group][32]
//   codes, then fp32 scales [pass][token][group]) from global memory, each
//   lane its own B fragments (up to 32 tokens);
// * a8_tiled_lds<STAGE = true> copies a filled workspace into LDS once per
//   workgroup (up to 16 tokens where the copy fits one round of loads and the
//   LDS keeps the shape's workgroups resident), and its waves read their B
//   fragments from LDS: the per-lane 8- and 4-byte fragment loads of the
//   first form, repeated by every workgroup, become one coalesced copy;
// * a8_tiled_lds<STAGE = false> (a8_tiled_fused; up to 16 tokens, k % 8 == 0,
//   its activations within 64 KB of LDS) quantizes the fp16 activations
//   itself: each workgroup issues its first two weight batches, quantizes
//   every token's groups into LDS with the quantizer's arithmetic (workgroup 0
//   also writes them to the workspace, so the workspace ends as the quantizer
//   leaves it), and reads its B fragments from LDS. One launch replaces the
//   quantizer's and the projection's.
// The group sums and their order depend only on the workgroup shape, which
// all three take from one table: at one shape they give the same bytes.
//
// Launch: W waves over RB row blocks per workgroup, the chunks split evenly
// over the waves, two batches of one chunk in flight per wave (the loads are
// unconditional and the loop's entry and back edge leave the same requests
// outstanding, so each multiply waits only for its own batch); the W partial
// tiles are summed through LDS in wave order, so results are deterministic.
#include "a8_group.hpp"

#include <algorithm>
#include <type_traits>

namespace vt {
namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));

// Runs a wave's `batches` multiplies with NBUF batches in flight: buf[j]
// holds batch j on entry, and batch i + NBUF is requested into batch i's
// buffer as soon as batch i is multiplied. The steady loop requests
// unconditionally (every wait then covers only the batch about to be
// multiplied) and multiplies with the second-group check off
// (consume(batch, std::false_type)); the tail, the last NBUF .. 2 * NBUF - 1
// batches, which hold the wave's last chunk, checks (std::true_type).
template <int NBUF, class Batch, class Fetch, class Consume>
__device__ __forceinline__ void run_pipeline(int batches, Batch (&buf)[NBUF], Fetch& fetch, Consume& consume) {
    int i = 0;
    for (; i + 2 * NBUF - 1 < batches; i += NBUF) {
#pragma unroll
        for (int j = 0; j < NBUF; ++j) {
            consume(buf[j], std::false_type{});
            __builtin_amdgcn_sched_barrier(0);
            fetch(i + NBUF + j, buf[j]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Here batches - i < 2 * NBUF: at most batches i + NBUF .. i + 2 * NBUF - 2
    // remain to be requested.
#pragma unroll
    for (int j = 0; j < NBUF; ++j) {
        if (i + j < batches) consume(buf[j], std::true_type{});
        if (j < NBUF - 1 && i + NBUF + j < batches) fetch(i + NBUF + j, buf[j]);
    }
#pragma unroll
    for (int j = 0; j < NBUF - 1; ++j)
        if (i + NBUF + j < batches) consume(buf[j], std::true_type{});
}

template <int RB, int NB, int P>
struct A8Batch {
    uint4 w[RB];              // 16 weight code bytes per block (groups 2c and 2c + 1)
    uint4 ws[RB];             // four rows' scale pairs (fp16)
    uint2 ac[P][NB][2];       // 8 activation code bytes of groups 2c and 2c + 1
    float as[P][NB][2];       // the token's activation scales of the two groups
    bool pair;                // group 2c + 1 exists (false only in the last chunk of an odd group count)
};

template <int W, int RB, int NB, int P, int NBUF>
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

    // Only a wave's last chunk can lack its second group, and it is one of the
    // loop's tail multiplies: the loop body takes the group unconditionally.
    auto consume = [&](const A8Batch<RB, NB, P>& t, auto last) {
        const bool second = !decltype(last)::value || t.pair;
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
                        if (second)
                            y[b][tb][e] = fmaf(static_cast<float>(db[0][e]), wsb * t.as[0][tb][1], y[b][tb][e]);
                    } else {
                        const float ta = fmaf(static_cast<float>(da[1][e]), t.as[1][tb][0],
                                              static_cast<float>(da[0][e]) * t.as[0][tb][0]);
                        const float tbv = fmaf(static_cast<float>(db[1][e]), t.as[1][tb][1],
                                               static_cast<float>(db[0][e]) * t.as[0][tb][1]);
                        y[b][tb][e] = fmaf(ta, wsa, y[b][tb][e]);
                        if (second) y[b][tb][e] = fmaf(tbv, wsb, y[b][tb][e]);
                    }
                }
            }
        }
    };

    if (batches > 0) {
        A8Batch<RB, NB, P> buf[NBUF];
#pragma unroll
        for (int j = 0; j < NBUF; ++j) fetch(j, buf[j]);
        run_pipeline<NBUF>(batches, buf, fetch, consume);
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

// Bytes of LDS rows in a8_tiled_fused: a (pass, token) code row holds the
// groups' 32 codes plus 32 bytes of padding (rows of consecutive tokens start
// on different banks); a scale row holds an even number of floats, two more
// than the groups rounded up to even (the pair of a chunk is one 8-byte read).
__host__ __device__ constexpr int a8_code_row(int groups) { return 32 * groups + 32; }
__host__ __device__ constexpr int a8_scale_row(int groups) { return 2 * ((groups + 1) / 2) + 2; }
// Quantizer tasks (4 per group and token) per thread of a8_tiled_fused: the
// workgroup quantizes all activations in one round of loads.
constexpr int kA8FusedTasks = 3;
// Workspace units (16 bytes of codes) and scales per thread of the staging
// form: every admitted launch copies its activations in one round of loads.
constexpr int kA8StageUnits = 10, kA8StageScales = 8;

// The idle pattern of an exchange slot: both fp32 halves a signalling NaN,
// which no arithmetic result takes (the pattern venturi_q8_tiled_workspace_init
// writes).
constexpr unsigned long long kA8SlotIdle = 0x7f8000017f800001ull;

// Stores lane (q, r)'s outputs: rows 16 blk + 4q .. +3 of token r. KS == 2:
// the tile is one of two K halves; the lane exchanges its row pairs (4q, 4q+1)
// and (4q+2, 4q+3) with two 64-bit slots of (r, blk, q): the first half to
// arrive finds the idle pattern and leaves its pair, the second adds the
// other pair (a sum of two fp32 terms, the same whichever arrives first),
// re-arms the slot and stores. Only the slot is shared: no fence, no waiting.
template <int KS>
__device__ __forceinline__ void a8_finish(__half* __restrict__ out, unsigned long long* __restrict__ slots,
                                          const float4v& sum, int blk, int q, int r, int tokens, int n, int blocks) {
    if (r >= tokens) return;
    __half* o = out + static_cast<std::int64_t>(r) * n + 16 * blk + 4 * q;
    const int row0 = 16 * blk + 4 * q;
    if constexpr (KS == 1) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (row0 + e < n) o[e] = from_f32<__half>(sum[e]);
    } else {
        static_assert(KS == 2, "K is split in two at most");
        unsigned long long* slot = slots + ((static_cast<std::int64_t>(r) * blocks + blk) * 4 + q) * 2;
        unsigned long long old[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const unsigned long long packed = (static_cast<unsigned long long>(__float_as_uint(sum[2 * h + 1])) << 32) |
                                              __float_as_uint(sum[2 * h]);
            old[h] = __hip_atomic_exchange(slot + h, packed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (old[h] == kA8SlotIdle) continue;
            __hip_atomic_store(slot + h, kA8SlotIdle, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float lo = sum[2 * h] + __uint_as_float(static_cast<std::uint32_t>(old[h]));
            const float hi = sum[2 * h + 1] + __uint_as_float(static_cast<std::uint32_t>(old[h] >> 32));
            if (row0 + 2 * h < n) o[2 * h] = from_f32<__half>(lo);
            if (row0 + 2 * h + 1 < n) o[2 * h + 1] = from_f32<__half>(hi);
        }
    }
}

template <int RB, int P>
struct FusedBatch {
    uint4 w[RB];   // 16 weight code bytes per block (groups 2c and 2c + 1)
    uint4 ws[RB];  // four rows' scale pairs (fp16)
    uint2 xa[P];   // the lane's 8 activation code bytes of group 2c (from LDS)
    uint2 xb[P];   // ... of group 2c + 1
    float2 as[P];  // the token's activation scales of the two groups (from LDS)
    int ch;        // the chunk
};

// STAGE = false: a8_tiled_fused, the activations quantized from x (and
// written to the workspace by workgroup 0). STAGE = true: the activations
// copied from a filled workspace (acodes, ascales) into the same LDS rows.
// KS == 2 (staged form only): workgroups 2g and 2g + 1 take the first and
// second half of row-block group g's chunks; LDS holds only the half's groups
// and the two partial tiles meet through the slots (a8_finish).
template <int W, int RB, int P, int NBUF, bool STAGE, int KS>
__global__ __launch_bounds__(W * 64) void a8_tiled_lds(const __half* x, const std::int8_t* __restrict__ acodes,
                                                       const float* __restrict__ ascales, std::int8_t* __restrict__ wcodes,
                                                       float* __restrict__ wscales, const uint4* __restrict__ codes,
                                                       const uint4* __restrict__ scales, __half* __restrict__ out,
                                                       unsigned long long* __restrict__ slots, int tokens, int n, int k,
                                                       int groups, int chunks, int blocks) {
    static_assert(KS == 1 || (KS == 2 && STAGE), "only the staged form splits K");
    extern __shared__ __align__(16) unsigned char lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int block0 = static_cast<int>(blockIdx.x / KS) * RB;
    const int used = (groups + 1) / 2;
    const int kper = (used + KS - 1) / KS;
    const int k0 = KS == 1 ? 0 : min(static_cast<int>(blockIdx.x % KS) * kper, used);
    const int k1 = min(k0 + kper, used);  // the workgroup's chunks [k0, k1), k0 < k1 (the host splits only long K)
    const int per = (k1 - k0 + W - 1) / W;
    const int c0 = min(k0 + wave * per, k1), c1 = min(c0 + per, k1);
    const int batches = c1 - c0;
    const int lg = KS == 1 ? groups : 2 * kper;  // groups an LDS row holds
    const int rs = a8_code_row(lg), ss = a8_scale_row(lg);
    std::int8_t* lcodes = reinterpret_cast<std::int8_t*>(lds);
    float* lscales = reinterpret_cast<float*>(lds + static_cast<std::size_t>(P) * tokens * rs);

    const uint4* wsrc[RB];
    const uint4* ssrc[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const std::int64_t blk = min(block0 + b, blocks - 1);  // clamped blocks are never stored
        wsrc[b] = codes + blk * chunks * 64 + lane;
        ssrc[b] = scales + blk * chunks * 4 + q;
    }
    // B fragments of this lane's token (absent tokens read the last token's
    // row and feed only outputs that are never stored).
    const int tr = min(r, tokens - 1);
    const std::int8_t* xrow[P];
    const float* srow[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        xrow[p] = lcodes + (p * tokens + tr) * rs + 8 * q;
        srow[p] = lscales + (p * tokens + tr) * ss;
    }
    // Chunk i of the wave, clamped to the wave's last chunk (a wave without
    // chunks reads chunk used - 1 and multiplies nothing): weights from
    // global memory, activations from LDS. In the last chunk of an odd group
    // count the second group is not the workspace's: its LDS bytes are not
    // written and its term is skipped.
    auto fetch_weights = [&](int i, FusedBatch<RB, P>& t) {
        t.ch = min(c0 + i, c1 - 1);
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            t.w[b] = stream_load(wsrc[b] + static_cast<std::int64_t>(t.ch) * 64);
            t.ws[b] = stream_load(ssrc[b] + static_cast<std::int64_t>(t.ch) * 4);
        }
    };
    auto fetch_activations = [&](FusedBatch<RB, P>& t) {
        const int lc = t.ch - k0;  // the chunk within the workgroup's LDS rows
#pragma unroll
        for (int p = 0; p < P; ++p) {
            t.xa[p] = *reinterpret_cast<const uint2*>(xrow[p] + 64 * lc);
            t.xb[p] = *reinterpret_cast<const uint2*>(xrow[p] + 64 * lc + 32);
            t.as[p] = *reinterpret_cast<const float2*>(srow[p] + 2 * lc);
        }
    };
    // Quantize every token's groups into LDS: 4 lanes per group, 8 columns
    // each (k % 8 == 0, so a lane's columns are all inside the row or all past
    // it), at most kA8FusedTasks tasks per thread (the host admits only such
    // launches). Their loads are unconditional (clamped addresses, masked
    // values) and go out before the first NBUF weight batches, so those are in
    // flight while the activations are quantized (and, counted in order, the
    // activation loads are not held behind them).
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const int tasks = tokens * groups * 4;
    FusedBatch<RB, P> buf[NBUF];
    if constexpr (STAGE) {
        // Copy: the codes as 16-byte units of the (pass, token) rows, the
        // scales one by one; at most kA8StageUnits / kA8StageScales per thread
        // (the host admits only such launches), all loads before the weights'.
        // The workgroup's groups [2 k0, g1) of every (pass, token) row.
        const int g1 = min(2 * k1, groups), gv = g1 - 2 * k0;
        const int units = P * tokens * gv * 2, nscales = P * tokens * gv;
        const uint4* src = reinterpret_cast<const uint4*>(acodes);
        uint4 u[kA8StageUnits];
        float sv[kA8StageScales];
#pragma unroll
        for (int j = 0; j < kA8StageUnits; ++j) {
            const int i = min(static_cast<int>(threadIdx.x) + j * W * 64, units - 1);
            const int row = i / (2 * gv);
            u[j] = src[(row * groups + 2 * k0) * 2 + (i - row * 2 * gv)];
        }
#pragma unroll
        for (int j = 0; j < kA8StageScales; ++j) {
            const int i = min(static_cast<int>(threadIdx.x) + j * W * 64, nscales - 1);
            const int row = i / gv;
            sv[j] = ascales[row * groups + 2 * k0 + (i - row * gv)];
        }
        __asm__ __volatile__("" ::: "memory");  // keeps these loads here, ahead of the weights'
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NBUF; ++j) fetch_weights(j, buf[j]);
#pragma unroll
        for (int j = 0; j < kA8StageUnits; ++j) {
            const int i = threadIdx.x + j * W * 64;
            if (i < units) {
                const int row = i / (2 * gv);
                *reinterpret_cast<uint4*>(lcodes + row * rs + (i - row * 2 * gv) * 16) = u[j];
            }
        }
#pragma unroll
        for (int j = 0; j < kA8StageScales; ++j) {
            const int i = threadIdx.x + j * W * 64;
            if (i < nscales) {
                const int row = i / gv;
                lscales[row * ss + (i - row * gv)] = sv[j];
            }
        }
    } else {
        uint4 u[kA8FusedTasks];
#pragma unroll
        for (int j = 0; j < kA8FusedTasks; ++j) {
            const int task = min(static_cast<int>(threadIdx.x) + j * W * 64, tasks - 1);
            const int gi = task >> 2, t = gi / groups, col = 32 * (gi - t * groups) + 8 * (task & 3);
            u[j] = *reinterpret_cast<const uint4*>(x + static_cast<std::int64_t>(t) * k + min(col, k - 8));
        }
        __asm__ __volatile__("" ::: "memory");  // keeps these loads here, ahead of the weights'
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NBUF; ++j) fetch_weights(j, buf[j]);
#pragma unroll
        for (int j = 0; j < kA8FusedTasks; ++j) {
            const int task = threadIdx.x + j * W * 64;
            if (task >= tasks) break;  // the 4 lanes of a group stop together
            const int sub = task & 3, gi = task >> 2;
            const int t = gi / groups, g = gi - t * groups;
            const bool inside = 32 * g + 8 * sub < k;
            float v[8] = {half_lo(u[j].x), half_hi(u[j].x), half_lo(u[j].y), half_hi(u[j].y),
                          half_lo(u[j].z), half_hi(u[j].z), half_lo(u[j].w), half_hi(u[j].w)};
            bool bad = false;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[e] = inside ? v[e] : 0.0f;
                bad |= !isfinite(v[e]);
            }
            const bool invalid = group_invalid<4>(bad);
#pragma unroll
            for (int p = 0; p < P; ++p) {
                std::uint32_t word[2];
                const float sc = quantize_pass<8, 4>(v, invalid, word);
                const uint2 pair = make_uint2(word[0], word[1]);
                *reinterpret_cast<uint2*>(lcodes + (p * tokens + t) * rs + 32 * g + 8 * sub) = pair;
                if (sub == 0) lscales[(p * tokens + t) * ss + g] = sc;
                if (blockIdx.x == 0) {
                    *reinterpret_cast<uint2*>(wcodes + (p * count + gi) * 32 + 8 * sub) = pair;
                    if (sub == 0) wscales[p * count + gi] = sc;
                }
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NBUF; ++j) fetch_activations(buf[j]);

    float4v y[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) y[b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    const int4v zero = {0, 0, 0, 0};

    // Only a wave's last chunk can lack its second group, and it is one of the
    // loop's tail multiplies: the loop body takes the group unconditionally.
    auto consume = [&](const FusedBatch<RB, P>& t, auto last) {
        const bool second = !decltype(last)::value || 2 * t.ch + 1 < groups;
        long xa[P], xb[P];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            xa[p] = static_cast<long>(static_cast<unsigned long>(t.xa[p].x) | (static_cast<unsigned long>(t.xa[p].y) << 32));
            xb[p] = static_cast<long>(static_cast<unsigned long>(t.xb[p].x) | (static_cast<unsigned long>(t.xb[p].y) << 32));
        }
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            const long wa = static_cast<long>(static_cast<unsigned long>(t.w[b].x) | (static_cast<unsigned long>(t.w[b].y) << 32));
            const long wb = static_cast<long>(static_cast<unsigned long>(t.w[b].z) | (static_cast<unsigned long>(t.w[b].w) << 32));
            const std::uint32_t wpair[4] = {t.ws[b].x, t.ws[b].y, t.ws[b].z, t.ws[b].w};
            int4v da[P], db[P];
#pragma unroll
            for (int p = 0; p < P; ++p) {
                da[p] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wa, xa[p], zero, 0, 0, 0);
                db[p] = __builtin_amdgcn_mfma_i32_16x16x32_i8(wb, xb[p], zero, 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float wsa = half_lo(wpair[e]), wsb = half_hi(wpair[e]);
                if constexpr (P == 1) {
                    y[b][e] = fmaf(static_cast<float>(da[0][e]), wsa * t.as[0].x, y[b][e]);
                    if (second) y[b][e] = fmaf(static_cast<float>(db[0][e]), wsb * t.as[0].y, y[b][e]);
                } else {
                    const float ta = fmaf(static_cast<float>(da[1][e]), t.as[1].x, static_cast<float>(da[0][e]) * t.as[0].x);
                    const float tbv = fmaf(static_cast<float>(db[1][e]), t.as[1].y, static_cast<float>(db[0][e]) * t.as[0].y);
                    y[b][e] = fmaf(ta, wsa, y[b][e]);
                    if (second) y[b][e] = fmaf(tbv, wsb, y[b][e]);
                }
            }
        }
    };
    auto fetch = [&](int i, FusedBatch<RB, P>& t) {
        fetch_weights(i, t);
        fetch_activations(t);
    };

    if (batches > 0) run_pipeline<NBUF>(batches, buf, fetch, consume);
    __syncthreads();  // every wave is done with the activations: LDS now holds the partial tiles
    float4v* partial = reinterpret_cast<float4v*>(lds);
#pragma unroll
    for (int b = 0; b < RB; ++b) partial[(wave * RB + b) * 64 + lane] = y[b];
    __syncthreads();
    for (int b = wave; b < RB; b += W) {
        float4v sum = partial[b * 64 + lane];
        for (int w = 1; w < W; ++w) {
            const float4v v = partial[(w * RB + b) * 64 + lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) sum[e] += v[e];
        }
        const int blk = block0 + b;
        if (blk < blocks) a8_finish<KS>(out, slots, sum, blk, q, r, tokens, n, blocks);
    }
}

// Workgroup shape of both kernels (unsplit K): W waves over RB row blocks,
// NBUF batches in flight per wave. Two token blocks take 8 waves over two row
// blocks (the other shapes spill); one token block takes 16 waves over one
// row block up to 256 blocks, over two up to 511 (grids of at most 256
// workgroups, one per CU), else 8 waves over three.
struct A8Shape {
    int waves, rb, nbuf;
    int ks = 1;  // workgroups splitting K (2: the staged form's halves, exchanging through slots)
};

A8Shape a8_shape(int token_blocks, int blocks) {
    if (token_blocks == 2) return {8, 2, 2};
    return blocks <= 256 ? A8Shape{16, 1, 2} : blocks <= 511 ? A8Shape{16, 2, 2} : A8Shape{8, 3, 2};
}

template <int W, int RB, int NBUF, int KS = 1>
struct ShapeTag {
    static constexpr int waves = W, rb = RB, nbuf = NBUF, ks = KS;
};

// Calls f(ShapeTag) for the compiled shape equal to sh.
template <class... Tags, class F>
void visit_shape(const A8Shape& sh, F&& f) {
    const bool found = ((sh.waves == Tags::waves && sh.rb == Tags::rb && sh.nbuf == Tags::nbuf && sh.ks == Tags::ks
                             ? (f(Tags{}), true)
                             : false) ||
                        ...);
    require(found, "internal: A8 decode shape not compiled");
}

template <class F>
void visit_one_block_shape(const A8Shape& sh, F&& f) {
    visit_shape<ShapeTag<16, 1, 2>, ShapeTag<16, 2, 2>, ShapeTag<8, 3, 2>>(sh, f);
}

template <int NB, int P>
void dispatch_a8_tiled(const std::int8_t* acodes, const float* ascales, const uint4* codes, const uint4* scales,
                       __half* out, int tokens, int n, int groups, int chunks, int blocks, hipStream_t stream) {
    auto launch = [&](auto tag) {
        using T = decltype(tag);
        a8_tiled_decode<T::waves, T::rb, NB, P, T::nbuf><<<(blocks + T::rb - 1) / T::rb, T::waves * 64, 0, stream>>>(
            acodes, ascales, codes, scales, out, tokens, n, groups, chunks, blocks);
    };
    const A8Shape sh = a8_shape(NB, blocks);
    if constexpr (NB == 2) visit_shape<ShapeTag<8, 2, 2>>(sh, launch);
    else visit_one_block_shape(sh, launch);
}

// LDS bytes of a8_tiled_lds: the activation rows of the workgroup's groups
// (all of them, or a K half's), later reused for the partial tiles.
std::size_t a8_lds_bytes(int tokens, int groups, int passes, const A8Shape& sh) {
    const int lg = sh.ks == 1 ? groups : 2 * (((groups + 1) / 2 + 1) / 2);
    const std::size_t act = static_cast<std::size_t>(passes) * tokens *
                            (a8_code_row(lg) + 4 * static_cast<std::size_t>(a8_scale_row(lg)));
    return std::max(act, static_cast<std::size_t>(sh.waves) * sh.rb * 64 * sizeof(float4v));
}

template <int P, bool STAGE>
void dispatch_a8_lds(const A8Shape& sh, const __half* x, const std::int8_t* acodes, const float* ascales,
                     std::int8_t* wcodes, float* wscales, const uint4* codes, const uint4* scales, __half* out,
                     unsigned long long* slots, int tokens, int n, int k, int groups, int chunks, int blocks,
                     std::size_t lds, hipStream_t stream) {
    auto launch = [&](auto tag) {
        using T = decltype(tag);
        auto* kernel = a8_tiled_lds<T::waves, T::rb, P, T::nbuf, STAGE, T::ks>;
        if (lds > 64 * 1024) {
            static const hipError_t raised = hipFuncSetAttribute(
                reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            check(raised);
        }
        kernel<<<(blocks + T::rb - 1) / T::rb * T::ks, T::waves * 64, lds, stream>>>(
            x, acodes, ascales, wcodes, wscales, codes, scales, out, slots, tokens, n, k, groups, chunks, blocks);
    };
    if constexpr (STAGE)
        visit_shape<ShapeTag<16, 1, 2>, ShapeTag<16, 2, 2>, ShapeTag<8, 3, 2>, ShapeTag<16, 3, 2>,
                    ShapeTag<16, 3, 2, 2>>(sh, launch);
    else
        visit_one_block_shape(sh, launch);
}

constexpr std::size_t kA8FusedLdsMax = 64 * 1024;   // the default dynamic LDS limit of a launch
constexpr std::size_t kA8StageLdsMax = 160 * 1024;  // gfx950 LDS per workgroup

}  // namespace

std::uint64_t a8_bytes(int tokens, int k, int passes);
void a8_quantize_launch(const void* x, void* workspace, std::uint64_t available, int tokens, int k, int passes,
                        hipStream_t stream);

namespace {

void validate_a8_tiled(const void* workspace, std::uint64_t available, const void* codes, const void* scales,
                       const void* out, int tokens, int n, int k, int padded, int passes) {
    require(workspace && codes && scales && out, "null A8 operand");
    require(tokens > 0 && tokens <= 32, "the matrix-core A8 decode kernel takes 1..32 tokens");
    require(n > 0 && k > 0 && padded == padded_k(k), "invalid A8 projection geometry");
    require(passes == 1 || passes == 2, "A8 passes must be 1 or 2");
    require(static_cast<std::uint64_t>(tokens) * n < INT32_MAX, "A8 output count exceeds int32");
    require(available >= a8_bytes(tokens, k, passes), "invalid A8 workspace size");
    require(aligned(workspace, 16) && aligned(codes, 16) && aligned(scales, 16) && aligned(out, 2),
            "misaligned A8 operand (workspace and tiled planes need 16 bytes)");
}

// How a filled workspace is projected: the staged form (activations copied
// into LDS once per workgroup) where one token block, one round of copy loads
// per thread and the LDS fit (LDS that would not let two 8-wave workgroups
// share a CU goes to one 16-wave workgroup over the same row blocks; LDS past
// one workgroup's share of the CU splits K over two workgroups of 16 waves and
// three row blocks, which exchange their halves through slots, where that grid
// runs in at most two rounds of one workgroup per CU, or where rows of at
// least 128 chunks in 257-384 blocks would leave CUs idle), else the register
// form.
struct A8TiledPlan {
    bool staged;
    A8Shape shape;
    std::size_t lds;
};

A8TiledPlan a8_tiled_plan(int tokens, int n, int k, int passes) {
    const int groups = (k + 31) / 32, blocks = (n + 15) / 16;
    A8Shape sh = a8_shape(tokens <= 16 ? 1 : 2, blocks);
    if (tokens > 16) return {false, sh, 0};
    std::size_t lds = a8_lds_bytes(tokens, groups, passes, sh);
    if (sh.waves == 8 && lds > kA8StageLdsMax / 2) {
        sh = A8Shape{16, sh.rb, sh.nbuf};
        lds = a8_lds_bytes(tokens, groups, passes, sh);
    }
    if (lds > kA8StageLdsMax && (groups + 1) / 2 >= 2 * 16 && (blocks + 2) / 3 * 2 <= 512) {
        sh = A8Shape{16, 3, 2, 2};
        lds = a8_lds_bytes(tokens, groups, passes, sh);
    } else if (blocks > 256 && (blocks + 2) / 3 * 2 <= 256 && (groups + 1) / 2 >= 128) {
        // Long rows of 257-384 blocks split K as well: 2 * ceil(blocks / 3)
        // workgroups instead of ceil(blocks / 2) (down at 8 tokens: 214, not 160).
        sh = A8Shape{16, 3, 2, 2};
        lds = a8_lds_bytes(tokens, groups, passes, sh);
    }
    const long threads = sh.waves * 64L;
    const long rows_groups = 1L * passes * tokens * (sh.ks == 1 ? groups : 2 * (((groups + 1) / 2 + 1) / 2));
    const bool fits = lds <= (sh.waves == 16 ? kA8StageLdsMax : kA8StageLdsMax / 2) &&
                      2 * rows_groups <= kA8StageUnits * threads && rows_groups <= kA8StageScales * threads;
    if (fits) return {true, sh, lds};
    return {false, a8_shape(1, blocks), 0};
}

}  // namespace

std::uint64_t a8_tiled_slot_bytes(int tokens, int n, int k, int passes) {
    require(tokens > 0 && tokens <= 32 && n > 0 && k > 0 && (passes == 1 || passes == 2),
            "invalid A8 projection geometry");
    const A8TiledPlan plan = a8_tiled_plan(tokens, n, k, passes);
    return plan.staged && plan.shape.ks == 2 ? static_cast<std::uint64_t>(tokens) * ((n + 15) / 16) * 64 : 0;
}

void a8_tiled_launch(const void* workspace, std::uint64_t available, const void* codes, const void* scales, void* out,
                     int tokens, int n, int k, int padded, int passes, void* slots, std::uint64_t slot_bytes,
                     hipStream_t stream) {
    validate_a8_tiled(workspace, available, codes, scales, out, tokens, n, k, padded, passes);
    const int groups = (k + 31) / 32;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const auto* acodes = static_cast<const std::int8_t*>(workspace);
    const auto* ascales = reinterpret_cast<const float*>(acodes + count * 32 * passes);
    const auto* cp = static_cast<const uint4*>(codes);
    const auto* sp = static_cast<const uint4*>(scales);
    auto* op = static_cast<__half*>(out);
    const int chunks = padded / 64, blocks = (n + 15) / 16;
    const A8TiledPlan plan = a8_tiled_plan(tokens, n, k, passes);
    if (plan.staged) {
        auto* sl = static_cast<unsigned long long*>(slots);
        if (plan.shape.ks == 2)
            require(sl && aligned(sl, 8) && slot_bytes >= a8_tiled_slot_bytes(tokens, n, k, passes),
                    "this A8 projection splits K: pass its slot buffer (venturi_q8_a8_tiled_workspace_bytes)");
        if (passes == 1)
            dispatch_a8_lds<1, true>(plan.shape, nullptr, acodes, ascales, nullptr, nullptr, cp, sp, op, sl, tokens, n,
                                     k, groups, chunks, blocks, plan.lds, stream);
        else
            dispatch_a8_lds<2, true>(plan.shape, nullptr, acodes, ascales, nullptr, nullptr, cp, sp, op, sl, tokens, n,
                                     k, groups, chunks, blocks, plan.lds, stream);
        return;
    }
    if (tokens <= 16) {
        if (passes == 1) dispatch_a8_tiled<1, 1>(acodes, ascales, cp, sp, op, tokens, n, groups, chunks, blocks, stream);
        else dispatch_a8_tiled<1, 2>(acodes, ascales, cp, sp, op, tokens, n, groups, chunks, blocks, stream);
    } else {
        if (passes == 1) dispatch_a8_tiled<2, 1>(acodes, ascales, cp, sp, op, tokens, n, groups, chunks, blocks, stream);
        else dispatch_a8_tiled<2, 2>(acodes, ascales, cp, sp, op, tokens, n, groups, chunks, blocks, stream);
    }
}

void a8_tiled_linear_launch(const void* x, void* workspace, std::uint64_t available, const void* codes,
                            const void* scales, void* out, int tokens, int n, int k, int padded, int passes,
                            void* slots, std::uint64_t slot_bytes, hipStream_t stream) {
    validate_a8_tiled(workspace, available, codes, scales, out, tokens, n, k, padded, passes);
    require(x != nullptr && aligned(x, 2), "invalid A8 input");
    const int groups = (k + 31) / 32, chunks = padded / 64, blocks = (n + 15) / 16;
    // The fused kernel: one token block, whole 16-byte activation pieces, its
    // LDS within the default limit and every quantizer task in its one round.
    const A8Shape sh = a8_shape(1, blocks);
    const std::size_t lds = a8_lds_bytes(tokens, groups, passes, sh);
    if (tokens > 16 || k % 8 != 0 || !aligned(x, 16) || lds > kA8FusedLdsMax ||
        4L * tokens * groups > static_cast<long>(kA8FusedTasks) * sh.waves * 64) {
        a8_quantize_launch(x, workspace, available, tokens, k, passes, stream);
        a8_tiled_launch(workspace, available, codes, scales, out, tokens, n, k, padded, passes, slots, slot_bytes,
                        stream);
        return;
    }
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    auto* wcodes = static_cast<std::int8_t*>(workspace);
    auto* wscales = reinterpret_cast<float*>(wcodes + count * 32 * passes);
    const auto* xp = static_cast<const __half*>(x);
    const auto* cp = static_cast<const uint4*>(codes);
    const auto* sp = static_cast<const uint4*>(scales);
    auto* op = static_cast<__half*>(out);
    if (passes == 1)
        dispatch_a8_lds<1, false>(sh, xp, nullptr, nullptr, wcodes, wscales, cp, sp, op, nullptr, tokens, n, k, groups,
                                  chunks, blocks, lds, stream);
    else
        dispatch_a8_lds<2, false>(sh, xp, nullptr, nullptr, wcodes, wscales, cp, sp, op, nullptr, tokens, n, k, groups,
                                  chunks, blocks, lds, stream);
}

}  // namespace vt

// Extension: the W8A8 projection of venturi_q8_dp4a_run at 1..32 tokens on
// int8 matrix cores over the tiled Q8 planes (the layout of
// venturi_q8_tiled_run); same A8 workspace; outputs equal the reference's up
// to fp32 association (exact int32 group dots, groups summed in natural order).
// Shapes whose launch splits K take an exchange-slot buffer of
// venturi_q8_a8_tiled_workspace_bytes bytes, armed once with
// venturi_q8_tiled_workspace_init and left idle by every run.
extern "C" __attribute__((visibility("default"))) int venturi_q8_a8_tiled_run(
    const void* workspace, std::uint64_t available, const void* codes, const void* scales, void* out, int tokens,
    int n, int k, int padded, int passes, void* slots, std::uint64_t slot_bytes, void* stream) {
    return vt::guarded([&] {
        vt::a8_tiled_launch(workspace, available, codes, scales, out, tokens, n, k, padded, passes, slots, slot_bytes,
                            static_cast<hipStream_t>(stream));
    });
}

// Extension: venturi_q8_dp4a_quantize followed by venturi_q8_a8_tiled_run, in
// one launch where the activations fit the fused kernel (the workspace ends
// holding the quantized activations either way, and the outputs are the same
// bytes as the two calls').
extern "C" __attribute__((visibility("default"))) int venturi_q8_a8_tiled_linear_run(
    const void* x, void* workspace, std::uint64_t available, const void* codes, const void* scales, void* out,
    int tokens, int n, int k, int padded, int passes, void* slots, std::uint64_t slot_bytes, void* stream) {
    return vt::guarded([&] {
        vt::a8_tiled_linear_launch(x, workspace, available, codes, scales, out, tokens, n, k, padded, passes, slots,
                                   slot_bytes, static_cast<hipStream_t>(stream));
    });
}

// Extension: bytes of the exchange slots the two entry points above need for
// this shape (0 when its launch does not split K; 0 with a message on invalid
// geometry).
extern "C" __attribute__((visibility("default"))) std::uint64_t venturi_q8_a8_tiled_workspace_bytes(int tokens, int n,
                                                                                                   int k, int passes) {
    std::uint64_t bytes = 0;
    if (!vt::host_guarded([&] { bytes = vt::a8_tiled_slot_bytes(tokens, n, k, passes); })) return 0;
    return bytes;
}
