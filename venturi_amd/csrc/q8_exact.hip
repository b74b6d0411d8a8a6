// Q8 A16 projection in the reference's canonical floating-point order.
//
// Reference semantics (blocks.cu:306-321, q8_head; the tiled and warp-exact
// variants at :342-442 produce the same bytes): for output (t, n) there are 256
// "virtual threads" j; thread j accumulates, for c = j, j+256, ... < k,
//     acc_j = fmaf(x[t][c], f32(code[n][c]) * f32(scale[n][c/32]), acc_j)
// then each group of 32 virtual threads is summed by a shfl_down 16/8/4/2/1
// tree, and the eight group sums by the same tree over 32 lanes in which only
// lanes 0..7 are nonzero. The result is rounded once to the activation type.
//
// gfx950 mapping: one 64-lane wave owns all 256 virtual threads of a row;
// lane L holds j = 4L..4L+3, so one chunk of 256 columns is a single dword
// per lane (256 contiguous bytes per wave) and every virtual thread's FMA
// chain stays in one lane in increasing column order. The activations are
// staged in LDS (zero past k): streamed weights would otherwise evict them
// from the vector L1 and every chunk would re-read them from L2, which halves
// the achievable HBM rate. One and two tokens stage the whole token tile once
// per persistent workgroup; from three tokens, where the FMAs bind, the slab
// form stages K in slabs. The code*scale product is exact in fp32 (8-bit by
// 11-bit significands), so its evaluation order is immaterial.
#include "common.hpp"

#include <algorithm>
#include <type_traits>

namespace vt {
namespace {

constexpr int kWaves = 16;  // waves per 1024-thread workgroup
constexpr int kThreads = kWaves * 64;

// Accumulates one chunk of 256 columns (lane L: columns 4L..4L+3 of the
// chunk) for TT tokens and RR rows. Activations come from LDS, where columns
// at or beyond k hold +0: with finite weights they contribute
// fma(+0, w, acc) == acc exactly (accumulators start at +0 and a
// round-to-nearest sum is never -0), so they need no masking.
// Weight value code * scale for the four codes of a word, exactly: with
// u = code + 128 (code ^ 0x80 per byte), fmaf(f32(u), s, -128 s) has an exact
// product and addend whose exact sum code * s fits fp32, so it is returned
// unrounded; this is bit-identical to f32(code) * s and costs a byte convert
// and one FMA per weight.
template <int RR>
__device__ __forceinline__ void word_weights(const std::uint32_t (&cw)[RR], const float (&s)[RR], float (&w)[RR][4]) {
#pragma unroll
    for (int r = 0; r < RR; ++r) {
        const std::uint32_t u = cw[r] ^ 0x80808080u;
        const float bias = -128.0f * s[r];
#pragma unroll
        for (int v = 0; v < 4; ++v) w[r][v] = fmaf(static_cast<float>((u >> (8 * v)) & 0xFFu), s[r], bias);
    }
}

// One chunk: 4 consecutive columns per lane, acc = fmaf(x, code*scale, acc).
// Activations are staged as 4 x 16-bit words (uint2) or, for single-token
// tiles, as fp32 (float4) converted once when staged.
template <class T, int TT, int RR>
__device__ __forceinline__ void chunk_fma(const uint2* __restrict__ xs, int stride, const std::uint32_t (&cw)[RR],
                                          const float (&s)[RR], float (&acc)[TT][RR][4]) {
    float w[RR][4];
    word_weights<RR>(cw, s, w);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        const uint2 xw = xs[t * stride];
        float xv[4];
        if constexpr (std::is_same<T, __half>::value) {
            xv[0] = half_lo(xw.x); xv[1] = half_hi(xw.x); xv[2] = half_lo(xw.y); xv[3] = half_hi(xw.y);
        } else {
            xv[0] = bf16_lo(xw.x); xv[1] = bf16_hi(xw.x); xv[2] = bf16_lo(xw.y); xv[3] = bf16_hi(xw.y);
        }
#pragma unroll
        for (int r = 0; r < RR; ++r)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[t][r][v] = fmaf(xv[v], w[r][v], acc[t][r][v]);
    }
}

template <int RR>
__device__ __forceinline__ void chunk_fma_f32(const float4* __restrict__ xs, const std::uint32_t (&cw)[RR],
                                              const float (&s)[RR], float (&acc)[1][RR][4]) {
    float w[RR][4];
    word_weights<RR>(cw, s, w);
    const float4 x4 = *xs;
    const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
    for (int r = 0; r < RR; ++r)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[0][r][v] = fmaf(xv[v], w[r][v], acc[0][r][v]);
}

// Persistent waves. Wave w owns row blocks w, w+W, w+2W, ... (RR rows each);
// every row block is a sequence of tiles of U chunks, and a wave walks the
// flat sequence of its (row block, tile) pairs with a two-deep ping-pong
// prefetch: the code words and scales of tile i+1 are in flight while tile i
// is accumulated. Each virtual thread's chain still advances one chunk at a
// time in increasing column order, so the association is the canonical one.
template <int RR, int U>
struct Tile {
    std::uint32_t cw[U][RR];
    unsigned short sb[U][RR];
};

// SHIFT: the code plane starts `shift` (1..3) bytes past a 4-byte boundary
// (a row-offset view, which the reference accepts). `codes` then points at
// that boundary and every code word is assembled from two aligned words with
// v_alignbyte. The second word of a row's last code word holds the row's
// last `shift` bytes, so no load leaves the plane's allocation.
template <class T, int TT, int RR, int U, bool VEC, bool SHIFT>
__global__ __launch_bounds__(kThreads) void q8_exact(const T* __restrict__ x,
                                                const std::int8_t* __restrict__ codes,
                                                const __half* __restrict__ scales,
                                                T* __restrict__ out, int tokens, int n, int k,
                                                int padded, int shift) {
    // [TT][tiles*U*64] groups of 4 activations: 16-bit words, or fp32 when TT == 1.
    extern __shared__ uint4 xstage[];
    uint2* xs = reinterpret_cast<uint2*>(xstage);
    float4* xf = reinterpret_cast<float4*>(xstage);
    constexpr bool kF32X = TT == 1;
    const int lane = threadIdx.x & 63;
    const int chunks = (k + 255) >> 8;
    const int tiles = (chunks + U - 1) / U;
    const int stride = tiles * U * 64;
    const int t0 = blockIdx.y * TT;

    // Stage the token tile's activations; zero past k and past `tokens`.
    for (int t = 0; t < TT; ++t) {
        const bool live_token = t0 + t < tokens;
        const T* src = x + static_cast<std::int64_t>(min(t0 + t, tokens - 1)) * k;
        for (int i = threadIdx.x; i < stride; i += kThreads) {
            const int col = 4 * i;
            uint2 w = make_uint2(0u, 0u);
            if (live_token && col < k) {
                if (VEC) {
                    w = *reinterpret_cast<const uint2*>(src + col);
                } else {
                    const unsigned short* p = reinterpret_cast<const unsigned short*>(src);
                    unsigned short h[4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) h[v] = col + v < k ? p[col + v] : static_cast<unsigned short>(0);
                    w.x = h[0] | (static_cast<std::uint32_t>(h[1]) << 16);
                    w.y = h[2] | (static_cast<std::uint32_t>(h[3]) << 16);
                }
            }
            if constexpr (kF32X) {
                if constexpr (std::is_same<T, __half>::value)
                    xf[t * stride + i] = make_float4(half_lo(w.x), half_hi(w.x), half_lo(w.y), half_hi(w.y));
                else
                    xf[t * stride + i] = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
            } else {
                xs[t * stride + i] = w;
            }
        }
    }
    __syncthreads();

    // Wave-uniform quantities live in scalar registers, so every branch on
    // them below is a scalar branch and the prefetch is never predicated
    // (a predicated prefetch would make the compiler wait for it at once).
    // Workgroup-minor wave numbering: consecutive row blocks go to different
    // workgroups, so every workgroup (and CU) holds the same number of rows.
    const int wave = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) * gridDim.x + blockIdx.x);
    const int waves = gridDim.x * kWaves;
    const int blocks = (n + RR - 1) / RR;
    if (wave >= blocks) return;
    const int total = ((blocks - 1 - wave) / waves + 1) * tiles;
    const int groups = padded >> 5;
    const int full = k >> 8;                  // chunks whose 256 columns are all valid
    const int last_word = (padded >> 2) - 1;  // last code word of a row

    // Interior tiles address every chunk from one per-tile base with constant
    // offsets; the edge tile clamps its indices into the row. Weights read for
    // columns at or past k meet zero activations; clamped rows are computed
    // and never stored.
    auto fetch = [&](int i, Tile<RR, U>& tile) {
        const int block = wave + (i / tiles) * waves;
        const int c0 = (i % tiles) * U;
        const int row0 = block * RR;
#pragma unroll
        for (int r = 0; r < RR; ++r) {
            const std::int64_t row = min(row0 + r, n - 1);
            const std::uint32_t* wp = reinterpret_cast<const std::uint32_t*>(codes + row * padded);
            const unsigned short* sp = reinterpret_cast<const unsigned short*>(scales + row * groups);
            if (c0 + U <= full) {
                const std::uint32_t* wt = wp + c0 * 64 + lane;
                const unsigned short* st = sp + c0 * 8 + (lane >> 3);
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    if constexpr (SHIFT)
                        tile.cw[u][r] = __builtin_amdgcn_alignbyte(wt[u * 64 + 1], wt[u * 64], shift);
                    else
                        tile.cw[u][r] = wt[u * 64];
                    tile.sb[u][r] = st[u * 8];
                }
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int word = min((c0 + u) * 64 + lane, last_word);
                    if constexpr (SHIFT)
                        tile.cw[u][r] = __builtin_amdgcn_alignbyte(wp[word + 1], wp[word], shift);
                    else
                        tile.cw[u][r] = wp[word];
                    tile.sb[u][r] = sp[min((c0 + u) * 8 + (lane >> 3), groups - 1)];
                }
            }
        }
    };

    float acc[TT][RR][4];
    auto reset = [&] {
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int r = 0; r < RR; ++r)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][r][v] = 0.0f;
    };

    auto consume = [&](int i, const Tile<RR, U>& tile) {
        const int c0 = (i % tiles) * U;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float s[RR];
#pragma unroll
            for (int r = 0; r < RR; ++r) s[r] = __half2float(__ushort_as_half(tile.sb[u][r]));
            if constexpr (kF32X)
                chunk_fma_f32<RR>(xf + (c0 + u) * 64 + lane, tile.cw[u], s, acc);
            else
                chunk_fma<T, TT, RR>(xs + (c0 + u) * 64 + lane, stride, tile.cw[u], s, acc);
        }
        if (i % tiles == tiles - 1) {
            const int row0 = (wave + (i / tiles) * waves) * RR;
#pragma unroll
            for (int t = 0; t < TT; ++t)
#pragma unroll
                for (int r = 0; r < RR; ++r) {
                    const float y = canonical_sum(acc[t][r][0], acc[t][r][1], acc[t][r][2], acc[t][r][3]);
                    if (lane == 0 && t0 + t < tokens && row0 + r < n)
                        out[static_cast<std::int64_t>(t0 + t) * n + row0 + r] = from_f32<T>(y);
                }
            reset();
        }
    };

    // Ping-pong over the wave's tiles; the prefetch past the last tile re-reads
    // the last tile (unconditional, so the wait before each consume covers only
    // the older tile).
    reset();
    Tile<RR, U> a, b;
    fetch(0, a);
    for (int i = 0; i < total; i += 2) {
        fetch(min(i + 1, total - 1), b);
        consume(i, a);
        if (i + 1 >= total) break;
        fetch(min(i + 2, total - 1), a);
        consume(i + 1, b);
    }
}

// Multi-token form. A workgroup of W waves owns W*RR rows and a tile of TT
// tokens and walks K in slabs of S chunks: the tile's activations for one
// slab are staged in LDS as fp32 (two buffers, one barrier per slab) while
// every wave streams its RR rows' code words and scales for the next slab
// into registers. Each weight value code*scale is formed once and multiplied
// into TT tokens; each staged activation is read once per RR rows. The
// products are plain fp32 FMAs on fp32 operands: on MI355X v_fma_mix_f32 (an
// FMA taking an fp16 operand) issues at 0.6 of v_fma_f32's rate, so the
// activations are converted once when staged and the scales once per chunk.
// A virtual thread's FMA chain still advances one chunk at a time in
// increasing column order inside one lane, so the association is the
// canonical one, and the LDS footprint (2*TT*S KiB) does not grow with K.
template <int TT, int RR, int S, int W, int B>
struct SlabGeom {
    static constexpr int kThreads = W * 64;
    static constexpr int kUnits = TT * S * 64;          // 4-column activation units per slab
    static constexpr int kPer = kUnits / kThreads;      // units staged per thread
    static constexpr int kRed = B * 256;                // floats of one wave's reduction scratch
    static constexpr std::size_t kLds = 2 * kUnits * sizeof(float4) + W * kRed * sizeof(float);
    static_assert(kUnits % kThreads == 0, "whole activation units per thread");
    static_assert(B == 0 || B == 4 || B == 8, "outputs reduced together (0: one at a time in registers)");
    static_assert(B == 0 || (TT * RR) % B == 0, "whole batches of outputs");
};

template <int S, int RR>
struct SlabWeights {
    std::uint32_t cw[S][RR];
    unsigned short sb[S][RR];
};

template <class T, int TT, int RR, int S, int W, int B, bool VEC, bool SHIFT>
__global__ __launch_bounds__(W * 64) void q8_exact_slab(const T* __restrict__ x,
                                                       const std::int8_t* __restrict__ codes,
                                                       const __half* __restrict__ scales,
                                                       T* __restrict__ out, int tokens, int n, int k,
                                                       int padded, int shift) {
    using G = SlabGeom<TT, RR, S, W, B>;
    // Dynamic LDS: two activation slabs, then one reduction scratch per wave.
    extern __shared__ float4 slab_lds[];
    auto* xs = reinterpret_cast<float4(*)[G::kUnits]>(slab_lds);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float* red = reinterpret_cast<float*>(slab_lds + 2 * G::kUnits) + wave * G::kRed;
    const int t0 = blockIdx.y * TT;
    const int chunks = (k + 255) >> 8;
    const int slabs = (chunks + S - 1) / S;
    const int groups = padded >> 5;
    const int last_word = (padded >> 2) - 1;
    // Persistent workgroups: workgroup b owns row groups b, b + gridDim.x, ...
    // (W*RR rows each) and walks the flat sequence of its (row group, slab)
    // items, so the pipeline runs on across row groups.
    const int rgroups = (n + W * RR - 1) / (W * RR);
    const int total = ((rgroups - 1 - static_cast<int>(blockIdx.x)) / static_cast<int>(gridDim.x) + 1) * slabs;

    // Activation staging: unit i of a slab is token i / (S*64), columns
    // 4 * (i % (S*64)) .. +3 of the slab. Loads use clamped addresses and the
    // units past k or past `tokens` are zeroed when stored, so no load is
    // predicated (a predicated load would make the compiler wait for it at
    // once).
    uint2 xr[G::kPer];
    auto xload = [&](int slab) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < G::kPer; ++u) {
            const int i = tid + u * G::kThreads;
            const int t = min(t0 + i / (S * 64), tokens - 1);
            const int col = slab * S * 256 + 4 * (i % (S * 64));
            const T* src = x + static_cast<std::int64_t>(t) * k;
            if constexpr (VEC) {
                xr[u] = *reinterpret_cast<const uint2*>(src + min(col, k - 4));
            } else {
                const unsigned short* p = reinterpret_cast<const unsigned short*>(src);
                unsigned short h[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) h[v] = p[min(col + v, k - 1)];
                xr[u].x = h[0] | (static_cast<std::uint32_t>(h[1]) << 16);
                xr[u].y = h[2] | (static_cast<std::uint32_t>(h[3]) << 16);
            }
        }
    };
    auto xstore = [&](int slab, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < G::kPer; ++u) {
            const int i = tid + u * G::kThreads;
            const bool live_token = t0 + i / (S * 64) < tokens;
            const int col = slab * S * 256 + 4 * (i % (S * 64));
            uint2 w = xr[u];
            if constexpr (VEC) {
                if (!live_token || col >= k) w = make_uint2(0u, 0u);
            } else {
                const std::uint32_t m0 = live_token && col < k ? 0xffffu : 0u;
                const std::uint32_t m1 = live_token && col + 1 < k ? 0xffff0000u : 0u;
                const std::uint32_t m2 = live_token && col + 2 < k ? 0xffffu : 0u;
                const std::uint32_t m3 = live_token && col + 3 < k ? 0xffff0000u : 0u;
                w.x &= m0 | m1;
                w.y &= m2 | m3;
            }
            if constexpr (std::is_same<T, __half>::value)
                xs[buf][i] = make_float4(half_lo(w.x), half_hi(w.x), half_lo(w.y), half_hi(w.y));
            else
                xs[buf][i] = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
        }
    };
    // The RR rows' code words and scales of one slab of row group rg; indices
    // are clamped into the row (columns past k meet zero activations) and
    // rows past n are read again as row n-1 and never stored.
    auto wload = [&](int rg, int slab, SlabWeights<S, RR>& w) __attribute__((always_inline)) {
        const int row0 = (rg * W + wave) * RR;
#pragma unroll
        for (int r = 0; r < RR; ++r) {
            const std::int64_t row = min(row0 + r, n - 1);
            const std::uint32_t* wp = reinterpret_cast<const std::uint32_t*>(codes + row * padded);
            const unsigned short* sp = reinterpret_cast<const unsigned short*>(scales + row * groups);
#pragma unroll
            for (int u = 0; u < S; ++u) {
                const int c = slab * S + u;
                const int word = min(c * 64 + lane, last_word);
                if constexpr (SHIFT)
                    w.cw[u][r] = __builtin_amdgcn_alignbyte(stream_load(wp + word + 1), stream_load(wp + word), shift);
                else
                    w.cw[u][r] = stream_load(wp + word);
                w.sb[u][r] = stream_load(sp + min(c * 8 + (lane >> 3), groups - 1));
            }
        }
    };

    float acc[TT][RR][4];
    auto reset = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int r = 0; r < RR; ++r)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[t][r][v] = 0.0f;
    };
    // The first `live` chunks of the slab in `buf` (all S but in a row's
    // last slab).
    auto consume = [&](int buf, const SlabWeights<S, RR>& w, int live) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < S; ++u) {
            if (u >= live) break;
            float s[RR];
#pragma unroll
            for (int r = 0; r < RR; ++r) {
                s[r] = __half2float(__ushort_as_half(w.sb[u][r]));
                asm volatile("" : "+v"(s[r]));  // keep the conversion out of the FMAs (no v_fma_mix_f32)
            }
            float wv[RR][4];
            word_weights<RR>(w.cw[u], s, wv);
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const float4 x4 = xs[buf][t * S * 64 + u * 64 + lane];
                const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
                for (int r = 0; r < RR; ++r)
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[t][r][v] = fmaf(xv[v], wv[r][v], acc[t][r][v]);
            }
            __builtin_amdgcn_sched_barrier(0);  // one chunk at a time (bounds the registers of hoisted reads)
        }
    };
    // End of a row group: the canonical reduction of the wave's TT*RR
    // outputs, B at a time through the wave's own LDS scratch (no barrier:
    // one wave's LDS operations complete in order). Output o's 256 partials
    // are stored in virtual-thread order, reference warp w (lanes 8w..8w+7)
    // in floats o*256 + 32w .. +31 with its eight 16-byte segments rotated
    // by w (segment s of warp w at slot (s + w) % 8, so eight lanes reading
    // the same segment of eight warps hit distinct banks), and lane
    // (q, w) = (lane / 8, lane % 8) reads reference warp w of output q and
    // runs that warp's shfl_down 16/8/4/2/1
    // tree in registers (the same additions in the same order as
    // canonical_sum: j + 16, + 8, + 4 across lanes there, + 2, + 1 within
    // the lane); the eight warp sums of an output, in lanes 8q..8q+7, then
    // take the two exact zero additions and the +4 / +2 / +1 steps as DPP
    // row shifts inside their 16-lane row. About 7-12 instructions per
    // output instead of canonical_sum's 32. With B = 4 the upper half of the
    // wave repeats the lower half's work and stores nothing; B = 0 runs
    // canonical_sum per output and needs no scratch (shapes whose LDS then
    // keeps two workgroups per CU).
    auto finish = [&](int rg) __attribute__((always_inline)) {
        const int row0 = (rg * W + wave) * RR;
        if constexpr (B == 0) {
#pragma unroll
            for (int t = 0; t < TT; ++t)
#pragma unroll
                for (int r = 0; r < RR; ++r) {
                    const float y = canonical_sum(acc[t][r][0], acc[t][r][1], acc[t][r][2], acc[t][r][3]);
                    if (lane == 0 && t0 + t < tokens && row0 + r < n)
                        out[static_cast<std::int64_t>(t0 + t) * n + row0 + r] = from_f32<T>(y);
                }
            reset();
            return;
        }
        constexpr int kB = B == 0 ? 1 : B;
        const int q = (lane >> 3) % kB, w = lane & 7;
#pragma unroll
        for (int b = 0; b < (TT * RR) / kB; ++b) {
#pragma unroll
            for (int i = 0; i < kB; ++i) {
                const int o = b * kB + i, t = o / RR, r = o % RR;
                *reinterpret_cast<float4*>(red + i * 256 + (lane >> 3) * 32 + (((lane & 7) + (lane >> 3)) & 7) * 4) =
                    make_float4(acc[t][r][0], acc[t][r][1], acc[t][r][2], acc[t][r][3]);
            }
            const float* src = red + q * 256 + w * 32;
            float v[32];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 f = *reinterpret_cast<const float4*>(src + ((i + w) & 7) * 4);
                v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
            }
#pragma unroll
            for (int h = 16; h >= 1; h >>= 1)
#pragma unroll
                for (int j = 0; j < h; ++j) v[j] = v[j] + v[j + h];
            float y = (v[0] + 0.0f) + 0.0f;
            y += row_shl<4>(y);
            y += row_shl<2>(y);
            y += row_shl<1>(y);
            const int o = b * kB + q, t = o / RR, r = o % RR;
            if (w == 0 && (lane >> 3) < kB && t0 + t < tokens && row0 + r < n)
                out[static_cast<std::int64_t>(t0 + t) * n + row0 + r] = from_f32<T>(y);
        }
        reset();
    };

    // Two register sets of weights (ping-pong) and two LDS buffers: while
    // item i is multiplied, item i+1's activations and weights are in
    // flight (past the last item, the last item is fetched again and never
    // used); the activations are stored into the other buffer after the
    // multiply, then one barrier. The scheduling barriers keep the next
    // item's loads ahead of the multiply (the scheduler would otherwise sink
    // them to their use and expose their latency). (c_rg, c_slab) is the
    // item being multiplied, (p_rg, p_slab) the one after it.
    const int live_last = chunks - (slabs - 1) * S;
    int c_rg = blockIdx.x, c_slab = 0;
    int p_rg = blockIdx.x, p_slab = 0;
    auto advance = [&](int& rg, int& slab) __attribute__((always_inline)) {
        if (++slab == slabs) {
            slab = 0;
            rg += gridDim.x;
        }
    };
    // One item: prefetch, multiply, finish a row group, stage, barrier.
    auto step = [&](int i, int buf, const SlabWeights<S, RR>& cur, SlabWeights<S, RR>& nxt) __attribute__((always_inline)) {
        const bool more = i + 1 < total;
        const int f_rg = more ? p_rg : c_rg, f_slab = more ? p_slab : c_slab;
        xload(f_slab);
        wload(f_rg, f_slab, nxt);
        __builtin_amdgcn_sched_barrier(0);
        const bool end = c_slab == slabs - 1;
        consume(buf, cur, end ? live_last : S);
        if (end) finish(c_rg);
        xstore(f_slab, buf ^ 1);
        __syncthreads();
        advance(c_rg, c_slab);
        advance(p_rg, p_slab);
    };

    SlabWeights<S, RR> wa, wb;
    reset();
    xload(0);
    wload(c_rg, 0, wa);
    xstore(0, 0);
    __syncthreads();
    advance(p_rg, p_slab);
    for (int i = 0; i < total; i += 2) {
        step(i, 0, wa, wb);
        if (i + 1 >= total) break;
        step(i + 1, 1, wb, wa);
    }
}

// LDS bytes for TT tokens at width k with tiles of U chunks.
inline std::size_t exact_lds_bytes(int tt, int u, int k) {
    const int chunks = (k + 255) >> 8;
    const std::size_t group = tt == 1 ? sizeof(float4) : sizeof(uint2);  // single-token tiles stage fp32
    return static_cast<std::size_t>(tt) * ((chunks + u - 1) / u) * u * 64 * group;
}

constexpr std::size_t kMaxLds = 160 * 1024;  // gfx950 LDS per workgroup

template <class T, int TT, int RR, int U>
void launch_tile(const void* x, const std::int8_t* codes, const __half* scales, void* out,
                 int tokens, int n, int k, int padded, hipStream_t stream) {
    // At most two 16-wave workgroups per CU (256 CUs): each stages the
    // activations once and streams many rows; grid.y walks token tiles (each
    // re-streams the weights). Row blocks are dealt round-robin over the
    // workgroups, so all of them are used as soon as there are 512 blocks.
    const int blocks = (n + RR - 1) / RR;
    const int groups = std::min(blocks, 512);
    const dim3 grid(groups, (tokens + TT - 1) / TT);
    require(grid.y <= 65535, "token tiles exceed the launch grid");
    const std::size_t lds = exact_lds_bytes(TT, U, k);
    require(lds <= kMaxLds, "activation tile exceeds LDS");
    const bool vec = (k % 4 == 0) && aligned(x, 8);
    const int shift = static_cast<int>(reinterpret_cast<std::uintptr_t>(codes) & 3);
    const void* kernels[4] = {
        reinterpret_cast<const void*>(q8_exact<T, TT, RR, U, true, false>),
        reinterpret_cast<const void*>(q8_exact<T, TT, RR, U, false, false>),
        reinterpret_cast<const void*>(q8_exact<T, TT, RR, U, true, true>),
        reinterpret_cast<const void*>(q8_exact<T, TT, RR, U, false, true>),
    };
    if (lds > 64 * 1024) {
        // Raise the dynamic-LDS limit of every variant once per process.
        static const hipError_t raised = [&kernels] {
            hipError_t status = hipSuccess;
            for (const void* f : kernels) {
                const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                         static_cast<int>(kMaxLds));
                if (status == hipSuccess) status = e;
            }
            return status;
        }();
        check(raised);
    }
    const T* xp = static_cast<const T*>(x);
    T* op = static_cast<T*>(out);
    const std::int8_t* base = codes - shift;  // 4-byte aligned
    if (shift == 0) {
        if (vec) q8_exact<T, TT, RR, U, true, false><<<grid, kThreads, lds, stream>>>(xp, codes, scales, op, tokens, n, k, padded, 0);
        else q8_exact<T, TT, RR, U, false, false><<<grid, kThreads, lds, stream>>>(xp, codes, scales, op, tokens, n, k, padded, 0);
    } else {
        if (vec) q8_exact<T, TT, RR, U, true, true><<<grid, kThreads, lds, stream>>>(xp, base, scales, op, tokens, n, k, padded, shift);
        else q8_exact<T, TT, RR, U, false, true><<<grid, kThreads, lds, stream>>>(xp, base, scales, op, tokens, n, k, padded, shift);
    }
}

// GENERAL: whether the shape is also built for code planes that start off a
// 4-byte boundary and for activations read element-wise (k % 4 != 0 or x not
// 8-byte aligned); the 8 x 4 tiles spill in those forms, so such calls take
// the 8 x 2 tiles.
template <class T, int TT, int RR, int S, int W, int B, bool GENERAL = true>
void launch_slab(const void* x, const std::int8_t* codes, const __half* scales, void* out, int tokens, int n, int k,
                 int padded, hipStream_t stream) {
    // Persistent grid: as many workgroups per token tile as stay resident
    // together (occupancy x CUs, shared by the token tiles), at most one per
    // row group.
    using G = SlabGeom<TT, RR, S, W, B>;
    constexpr int kT = W * 64;
    const void* kernels[4] = {
        reinterpret_cast<const void*>(q8_exact_slab<T, TT, RR, S, W, B, true, false>),
        GENERAL ? reinterpret_cast<const void*>(q8_exact_slab<T, TT, RR, S, W, B, !GENERAL, false>) : nullptr,
        GENERAL ? reinterpret_cast<const void*>(q8_exact_slab<T, TT, RR, S, W, B, true, GENERAL>) : nullptr,
        GENERAL ? reinterpret_cast<const void*>(q8_exact_slab<T, TT, RR, S, W, B, !GENERAL, GENERAL>) : nullptr,
    };
    static const int capacity = [&kernels] {
        if (G::kLds > 64 * 1024)
            for (const void* f : kernels)
                if (f) check(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(G::kLds)));
        int device = 0, cus = 0, per = 0;
        check(hipGetDevice(&device));
        check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
        check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernels[0], kT, G::kLds));
        return std::max(1, cus * per);
    }();
    const int rgroups = (n + W * RR - 1) / (W * RR);
    const int tiles = (tokens + TT - 1) / TT;
    require(tiles <= 65535, "token tiles exceed the launch grid");
    const dim3 grid(std::max(1, std::min(rgroups, capacity / tiles)), tiles);
    const bool vec = (k % 4 == 0) && aligned(x, 8);
    const int shift = static_cast<int>(reinterpret_cast<std::uintptr_t>(codes) & 3);
    const T* xp = static_cast<const T*>(x);
    T* op = static_cast<T*>(out);
    const std::int8_t* base = codes - shift;  // 4-byte aligned
    if (shift == 0 && vec) {
        q8_exact_slab<T, TT, RR, S, W, B, true, false><<<grid, kT, G::kLds, stream>>>(xp, codes, scales, op, tokens, n, k, padded, 0);
    } else if constexpr (GENERAL) {
        if (shift == 0) q8_exact_slab<T, TT, RR, S, W, B, false, false><<<grid, kT, G::kLds, stream>>>(xp, codes, scales, op, tokens, n, k, padded, 0);
        else if (vec) q8_exact_slab<T, TT, RR, S, W, B, true, true><<<grid, kT, G::kLds, stream>>>(xp, base, scales, op, tokens, n, k, padded, shift);
        else q8_exact_slab<T, TT, RR, S, W, B, false, true><<<grid, kT, G::kLds, stream>>>(xp, base, scales, op, tokens, n, k, padded, shift);
    } else {
        throw Invalid("this exact-route shape is built for 4-byte aligned codes and vector activation loads only");
    }
}

template <class T>
void launch_exact(const void* x, const std::int8_t* codes, const __half* scales, void* out,
                  int tokens, int n, int k, int padded, hipStream_t stream) {
    // One and two tokens: the whole activation tile staged once per
    // persistent workgroup (the weight stream binds). From three tokens the
    // FMAs bind and the slab form runs them as plain fp32 FMAs: tiles of 4
    // tokens x 2 rows per wave, 8 x 2, and 8 x 4 (slabs of 4 chunks, batched
    // reductions) beyond 8 tokens (config-2 step on MI355X, QKV / o_proj /
    // gate+up / down: 4 tokens 22.6 / 23.5 / 70.6 / 58.5 -> 15.7 / 16.5 /
    // 55.2 / 36.9 us; 8 tokens 32.2 / 29.6 / 111.4 / 111.8 -> 21.3 / 23.3 /
    // 85.0 / 53.5; 16 tokens 64.0 / 60.0 / 203.3 / 222.1 -> 39.1 / 43.5 /
    // 160.0 / 107.8; same bytes). The slab form also serves widths whose
    // whole tile exceeds LDS.
    if (tokens == 1 && exact_lds_bytes(1, 4, k) <= kMaxLds)
        launch_tile<T, 1, 1, 4>(x, codes, scales, out, tokens, n, k, padded, stream);
    else if (tokens <= 2 && exact_lds_bytes(2, 4, k) <= kMaxLds)
        launch_tile<T, 2, 1, 4>(x, codes, scales, out, tokens, n, k, padded, stream);
    else if (tokens <= 4) launch_slab<T, 4, 2, 4, 8, 0>(x, codes, scales, out, tokens, n, k, padded, stream);
    else if (tokens <= 8 || (reinterpret_cast<std::uintptr_t>(codes) & 3) != 0 || k % 4 != 0 || !aligned(x, 8))
        launch_slab<T, 8, 2, 2, 8, 0>(x, codes, scales, out, tokens, n, k, padded, stream);
    else launch_slab<T, 8, 4, 4, 8, 8, false>(x, codes, scales, out, tokens, n, k, padded, stream);
}

// One thread per 8 columns of a token's row (one scale covers them: 8 divides
// 32): one 8-byte code load (byte loads when the codes are not 8-byte
// aligned), one scale, and one 16-byte store when the output row allows it
// (k % 8 == 0 and a 16-byte aligned output), else 2-byte stores. grid.y runs
// over tokens.
template <class T>
__global__ __launch_bounds__(256) void q8_embedding(const std::int8_t* __restrict__ codes,
                                                    const __half* __restrict__ scales,
                                                    const std::int64_t* __restrict__ ids, T* __restrict__ out,
                                                    int tokens, int vocab, int k, int padded, bool codes8,
                                                    bool out16) {
    // Reference: blocks.cu:293-304 (ids outside [0, vocab) read as zero rows).
    const int col = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (col >= k) return;
    for (int t = blockIdx.y; t < tokens; t += gridDim.y) {
        const std::int64_t row = ids[t];
        float v[8];
        if (row >= 0 && row < vocab) {
            const std::int8_t* c = codes + row * padded + col;  // col + 8 <= padded
            std::uint32_t lo, hi;
            if (codes8) {
                const uint2 w = *reinterpret_cast<const uint2*>(c);
                lo = w.x;
                hi = w.y;
            } else {
                lo = hi = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    lo |= static_cast<std::uint32_t>(static_cast<std::uint8_t>(c[i])) << (8 * i);
                    hi |= static_cast<std::uint32_t>(static_cast<std::uint8_t>(c[4 + i])) << (8 * i);
                }
            }
            const float scale = __half2float(scales[row * (padded / 32) + col / 32]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = sbyte(lo, i) * scale;
                v[4 + i] = sbyte(hi, i) * scale;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
        }
        T* o = out + static_cast<std::int64_t>(t) * k + col;
        if (out16 && col + 8 <= k) {
            std::uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const T a = from_f32<T>(v[2 * i]), b = from_f32<T>(v[2 * i + 1]);
                w[i] = static_cast<std::uint32_t>(__builtin_bit_cast(unsigned short, a)) |
                       (static_cast<std::uint32_t>(__builtin_bit_cast(unsigned short, b)) << 16);
            }
            *reinterpret_cast<uint4*>(o) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            for (int i = 0; i < 8 && col + i < k; ++i) o[i] = from_f32<T>(v[i]);
        }
    }
}

void validate_q8(const void* x, const void* codes, const void* scales, const void* out, int tokens,
                 int n, int k, int padded) {
    require(x && codes && scales && out, "null Q8 operand");
    require(tokens > 0 && n > 0 && k > 0, "Q8 geometry must be positive");
    require(padded == padded_k(k), "padded K must equal ceil(k/128)*128");
    require(static_cast<std::int64_t>(tokens) * n < INT32_MAX, "Q8 output count exceeds int32");
    require(aligned(scales, 2) && aligned(x, 2) && aligned(out, 2), "Q8 fp16/bf16 operands must be 2-byte aligned");
}

}  // namespace

void q8_exact_launch(const void* x, const std::int8_t* codes, const __half* scales, void* out,
                     int tokens, int n, int k, int padded, int dtype, hipStream_t stream) {
    validate_q8(x, codes, scales, out, tokens, n, k, padded);
    if (dtype == kF16) launch_exact<__half>(x, codes, scales, out, tokens, n, k, padded, stream);
    else if (dtype == kBF16) launch_exact<__hip_bfloat16>(x, codes, scales, out, tokens, n, k, padded, stream);
    else throw Invalid("Q8 supports FP16/BF16 activations");
}

}  // namespace vt

extern "C" {

// Reference: blocks.cu:935-948 (venturi_q8_head_run), canonical bytes.
__attribute__((visibility("default"))) int venturi_q8_head_run(const void* x, const std::int8_t* codes,
                                                              const __half* scales, void* out, int tokens,
                                                              int vocab, int k, int padded, int dtype,
                                                              void* stream) {
    return vt::guarded([&] {
        vt::q8_exact_launch(x, codes, scales, out, tokens, vocab, k, padded, dtype,
                            static_cast<hipStream_t>(stream));
    });
}

// Reference: blocks.cu:918-934 (venturi_q8_embedding_run).
__attribute__((visibility("default"))) int venturi_q8_embedding_run(const std::int8_t* codes,
                                                                   const __half* scales,
                                                                   const std::int64_t* ids, void* out,
                                                                   int tokens, int vocab, int k, int padded,
                                                                   int dtype, void* stream) {
    return vt::guarded([&] {
        vt::require(codes && scales && ids && out, "null Q8 embedding operand");
        vt::require(tokens > 0 && vocab > 0 && k > 0 && padded == vt::padded_k(k), "invalid Q8 embedding geometry");
        vt::require(dtype == vt::kF16 || dtype == vt::kBF16, "Q8 supports FP16/BF16 activations");
        const dim3 grid((k + 2047) / 2048, std::min(tokens, 65535));
        const bool codes8 = vt::aligned(codes, 8);
        const bool out16 = k % 8 == 0 && vt::aligned(out, 16);
        auto s = static_cast<hipStream_t>(stream);
        if (dtype == vt::kF16)
            vt::q8_embedding<<<grid, 256, 0, s>>>(codes, scales, ids, static_cast<__half*>(out), tokens, vocab, k,
                                                  padded, codes8, out16);
        else
            vt::q8_embedding<<<grid, 256, 0, s>>>(codes, scales, ids, static_cast<__hip_bfloat16*>(out), tokens,
                                                  vocab, k, padded, codes8, out16);
    });
}

}  // extern "C"
