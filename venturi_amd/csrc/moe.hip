// Q4 W4A16 on fp16 matrix cores: a grouped (routed-expert) GEMM, the plain
// W4/5/6A16 GEMMs (decode and prefill), plus the device routing and per-token
// combine of the routed-expert MoE.
//
// Weight contract (flash_next_q4.cu:7-14, quantization/linear.py:86-95):
// w = fp16_RNE(q * scale). In registers: the nibble u = q + 8 becomes the
// fp16 1024 + u by byte permutation with 0x64, a packed fp16 add of -1032
// gives q exactly, and a packed fp16 multiply by the group scale rounds
// q * scale once, which is the contract's value. Dot products accumulate in
// fp32 on v_mfma_f32_16x16x32_f16 (association differs from the reference's
// cuBLAS/F.linear, which it pins by tolerance only).
//
// MoE semantics (flash_next_moe.py:139-161, flash_next_q4.py:204-224):
// for each expert e in ascending order, over its routed tokens:
//   gate, up = (x @ Wgu_e^T).chunk(2)      fp16 outputs
//   h = fp16(fp16(silu(gate)) * up)
//   y = fp16(h @ Wd_e^T) ; v = fp16(y * score)
//   out[token] = fp16(out[token] + v)       out starts at +0
// Every (token, slot) product is independent of the other tokens in its
// expert's segment, so the routing kernel may place a token anywhere inside
// its segment; the combine adds each token's values in ascending expert order
// (ties in position order), which is the reference's index_add_ order.
#include "common.hpp"

#include <algorithm>
#include <type_traits>

namespace vt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kRows = 128;        // weight rows per expert tile
constexpr int kChunk = 256;       // K columns staged per iteration (128 code bytes per row)
constexpr int kXStride = 264;     // LDS halves per token row (256 + 8 pad)
constexpr int kMaxExperts = 1024;

enum Epilogue { kSwiGLU = 1, kScore = 2 };

// Eight signed nibbles (one code word: columns c..c+7, even columns in the
// low nibbles) -> eight fp16 weights fp16(q * s), in the K order
// c, c+2, c+4, c+6, c+1, c+3, c+5, c+7 (activations are staged in that order).
__device__ __forceinline__ half8 dequant8(std::uint32_t word, half2v s2) {
    const std::uint32_t u = word ^ 0x88888888u;     // nibble u = q + 8
    const std::uint32_t lo = u & 0x0F0F0F0Fu;       // columns c, c+2, c+4, c+6
    const std::uint32_t hi = (u >> 4) & 0x0F0F0F0Fu;  // columns c+1, c+3, c+5, c+7
    const half2v bias = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    half2v p[4];
    p[0] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u));
    p[1] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u));
    p[2] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u));
    p[3] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u));
    half8 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v q = p[i] + bias;  // exact: q in [-8, 7]
        const half2v v = q * s2;       // one fp16 rounding of q * s
        w[2 * i] = v[0];
        w[2 * i + 1] = v[1];
    }
    return w;
}

// The same eight weights from a pre-biased word (nibble = q + 8, stored so by
// the tiled bank): a mask-and-or per pair of nibbles 16 bits apart places u
// (low nibble) or 16u (high nibble) in the mantissa of 1024 (0x6400); q is
// then one exact fp16 add (low: h - 1032) or fma (high: h/16 - 72), and q * s
// the contract's single rounding. Columns come out as c, c+4, c+1, c+5, c+2,
// c+6, c+3, c+7 (activations staged by interleave_biased to match).
__device__ __forceinline__ half8 dequant8_biased(std::uint32_t u, half2v s2) {
    const std::uint32_t v = u >> 8;
    const half2v lo_bias = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const half2v sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    const half2v hi_bias = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
    const half2v a = __builtin_bit_cast(half2v, (u & 0x000F000Fu) | 0x64006400u);  // c, c+4
    const half2v b = __builtin_bit_cast(half2v, (u & 0x00F000F0u) | 0x64006400u);  // c+1, c+5 (times 16)
    const half2v c = __builtin_bit_cast(half2v, (v & 0x000F000Fu) | 0x64006400u);  // c+2, c+6
    const half2v d = __builtin_bit_cast(half2v, (v & 0x00F000F0u) | 0x64006400u);  // c+3, c+7 (times 16)
    const half2v q[4] = {a + lo_bias, b * sixteenth + hi_bias, c + lo_bias, d * sixteenth + hi_bias};  // exact
    half8 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v x = q[i] * s2;  // one fp16 rounding of q * s
        w[2 * i] = x[0];
        w[2 * i + 1] = x[1];
    }
    return w;
}

// dequant8_biased with its three bit constants held in registers: a VOP3
// v_and_or_b32 takes no literal, so with literal constants the compiler splits
// each mask-and-or into two instructions (17 instead of 13 per word).
struct BiasedMasks {
    std::uint32_t lo, hi, one;  // 0x000F000F, 0x00F000F0, 0x64006400
};

__device__ __forceinline__ BiasedMasks biased_masks() {
    BiasedMasks m{0x000F000Fu, 0x00F000F0u, 0x64006400u};
    asm volatile("" : "+v"(m.lo), "+v"(m.hi), "+v"(m.one));  // opaque: kept in VGPRs, not re-folded to literals
    return m;
}

__device__ __forceinline__ half8 dequant8_biased(std::uint32_t u, half2v s2, const BiasedMasks& m) {
    const std::uint32_t v = u >> 8;
    const half2v lo_bias = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const half2v sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    const half2v hi_bias = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
    const half2v a = __builtin_bit_cast(half2v, (u & m.lo) | m.one);
    const half2v b = __builtin_bit_cast(half2v, (u & m.hi) | m.one);
    const half2v c = __builtin_bit_cast(half2v, (v & m.lo) | m.one);
    const half2v d = __builtin_bit_cast(half2v, (v & m.hi) | m.one);
    const half2v q[4] = {a + lo_bias, b * sixteenth + hi_bias, c + lo_bias, d * sixteenth + hi_bias};  // exact
    half8 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v x = q[i] * s2;  // one fp16 rounding of q * s
        w[2 * i] = x[0];
        w[2 * i + 1] = x[1];
    }
    return w;
}

// Eight consecutive activations x0..x7 -> x0, x4, x1, x5, x2, x6, x3, x7
// (the column order of dequant8_biased).
__device__ __forceinline__ uint4 interleave_biased(uint4 v) {
    uint4 r;
    r.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
    r.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
    r.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
    r.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
    return r;
}

// Eight (4 + HB)-bit codes of a Q5 (HB = 1) / Q6 (HB = 2) row: the low
// nibbles as in dequant8 and `h` holding the 8 * HB upper bits of the eight
// columns (column c + j's at bit HB * j, the high plane's LSB-first stream).
// The upper bits are placed above each nibble, the sign bit of the
// (4 + HB)-bit code is flipped (u = q + 2^(3+HB)) and 1024 + u converts
// exactly as for Q4; fp16(q * s) is the one rounding. Same K order as dequant8.
template <int HB>
__device__ __forceinline__ half8 dequant8_high(std::uint32_t word, std::uint32_t h, half2v s2) {
    constexpr std::uint32_t mask = (1u << HB) - 1u;
    std::uint32_t lo = word & 0x0F0F0F0Fu;         // columns c, c+2, c+4, c+6
    std::uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;  // columns c+1, c+3, c+5, c+7
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        lo |= ((h >> (HB * 2 * j)) & mask) << (8 * j + 4);
        hi |= ((h >> (HB * (2 * j + 1))) & mask) << (8 * j + 4);
    }
    constexpr std::uint32_t flip = 0x01010101u << (3 + HB);
    lo ^= flip;
    hi ^= flip;
    const half2v bias = {static_cast<_Float16>(-1024.0f - (1 << (3 + HB))),
                         static_cast<_Float16>(-1024.0f - (1 << (3 + HB)))};
    half2v p[4];
    p[0] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u));
    p[1] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u));
    p[2] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u));
    p[3] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u));
    half8 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v q = p[i] + bias;  // exact: q in [-2^(3+HB), 2^(3+HB))
        const half2v v = q * s2;       // one fp16 rounding of q * s
        w[2 * i] = v[0];
        w[2 * i + 1] = v[1];
    }
    return w;
}

// Eight Q5 (HB = 1) / Q6 (HB = 2) columns c .. c+7 of the tiled copy: `u` is
// the word's nibbles in dequant8_biased's order (unbiased), `reg` the high
// register holding this word as its word jj. A pair's upper fields sit at
// bits o + (0, 8, 4, 12)[m] and 16 above (o = HB * jj), biased so that nibble
// and fields form u = q + 2^(3 + HB); each pair's two fields go to bit 4 of
// its fp16 halves (1024 + u) or to bit 8 (1024 + 16 u, the x16 form), one
// shift serving the pairs at +4 and +8. q = 1024 + u - 1024 - 2^(3+HB) and
// (1024 + 16 u) / 16 - 64 - 2^(3+HB) are exact; fp16(q * s) is the one rounding.
struct HighMasks {
    std::uint32_t four, eight;  // the fields' positions: bit 4 / bit 8 of each half
};

template <int HB>
__device__ __forceinline__ HighMasks high_masks() {
    constexpr std::uint32_t f = (1u << HB) - 1u;
    HighMasks m{(f << 4) * 0x10001u, (f << 8) * 0x10001u};
    asm volatile("" : "+v"(m.four), "+v"(m.eight));  // kept in VGPRs for v_and_or_b32
    return m;
}

template <int HB>
__device__ __forceinline__ half8 dequant8_biased_high(std::uint32_t u, std::uint32_t reg, int jj, half2v s2,
                                                      const BiasedMasks& m, const HighMasks& hm) {
    const std::uint32_t v = u >> 8;
    const int o = HB * jj;
    const std::uint32_t at4 = reg << (4 - o);  // pair (c, c+1): offset o
    const std::uint32_t mid = reg >> o;        // pairs (c+4, c+5) at o + 4 and (c+2, c+3) at o + 8
    const std::uint32_t at12 = reg >> (4 + o); // pair (c+6, c+7): offset o + 12
    // The nibble terms are opaque to the combiner, which would otherwise fold
    // the two mask-and-ors of a pair into two ands and a three-input or.
    std::uint32_t na = (u & m.lo) | m.one, nb = (u & m.hi) | m.one, nc = (v & m.lo) | m.one, nd = (v & m.hi) | m.one;
    asm("" : "+v"(na), "+v"(nb), "+v"(nc), "+v"(nd));
    const half2v a = __builtin_bit_cast(half2v, (at4 & hm.four) | na);
    const half2v b = __builtin_bit_cast(half2v, (mid & hm.eight) | nb);
    const half2v c = __builtin_bit_cast(half2v, (mid & hm.four) | nc);
    const half2v d = __builtin_bit_cast(half2v, (at12 & hm.eight) | nd);
    constexpr float bias = 1 << (3 + HB);
    const half2v lo_bias = {static_cast<_Float16>(-1024.0f - bias), static_cast<_Float16>(-1024.0f - bias)};
    const half2v sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    const half2v hi_bias = {static_cast<_Float16>(-64.0f - bias), static_cast<_Float16>(-64.0f - bias)};
    const half2v q[4] = {a + lo_bias, b * sixteenth + hi_bias, c + lo_bias, d * sixteenth + hi_bias};  // exact
    half8 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v x = q[i] * s2;  // one fp16 rounding of q * s
        w[2 * i] = x[0];
        w[2 * i + 1] = x[1];
    }
    return w;
}

// Eight consecutive activations x0..x7 -> x0, x2, x4, x6, x1, x3, x5, x7.
__device__ __forceinline__ uint4 interleave8(uint4 v) {
    uint4 r;
    r.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);
    r.y = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);
    r.z = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);
    r.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);
    return r;
}

__device__ __forceinline__ float silu(float g) { return __fdiv_rn(g, 1.0f + expf(-g)); }

// ---------------------------------------------------------------------------
// Tiled expert planes (built at upload): a matrix is cut into tiles of 128 rows
// x 256 columns, stored tile after tile in [row tile][chunk] order, so one
// workgroup's stage is 16 KB of contiguous codes. Inside a tile, row block w
// (16 rows, one wave) is 2 KB laid out [half h][lane l][16 bytes] with
// l = 16q + m: lane (m, q) gets the 32 code bytes of its row m for chunk
// columns [64q, 64q + 64) (group q) as two 1 KB contiguous wave loads. Scales:
// [row tile][chunk][w][l] fp16, one 128-byte wave load. For gate/up, row block
// w holds gate rows 8w..8w+7 of the tile's 64 (m < 8) and the matching up rows
// (m >= 8). Codes are stored pre-biased: every nibble holds q + 8 (the
// dequant then needs no sign fix). Padding rows and columns hold q = 0 and
// zero scales.
struct Q4Tiled {
    const __half* x;            // activation rows (x_stride halves apart)
    const int* gather;          // slot -> x row (null: slot itself)
    const uint4* codes;         // expert 0 tiled codes
    const __half* scales;       // expert 0 tiled scales
    std::int64_t code_stride;   // uint4 units between experts
    std::int64_t scale_stride;  // halves between experts
    const int* seg;             // [experts + 1] slot offsets
    const __half* score;        // per-slot fp16 factor (kScore)
    __half* out;                // out[slot][out_stride]
    int n, k, chunks, x_stride, out_stride, experts, row_tiles, half_rows;
    // Routing inside the gate/up launch (the ROUTE instantiation): each
    // workgroup ranks its expert's pairs itself; seg and gather are not read.
    const std::int64_t* ids;  // [pairs] expert ids
    const __half* scores;     // [pairs]
    int* seg_out;             // [experts + 1], written by part 0 of each expert
    int* status;              // invalid-id count, written by expert 0's part 0
    int* pair_slot;           // [pairs] (-1 for invalid ids)
    int* slot_token;          // [pairs]
    __half* slot_score;       // [pairs]
    int pairs, top_k;
};

constexpr int kTileCodes = 8 * 128;  // uint4 per (tile, chunk): 8 row blocks x 2 KB

// Largest pair count routed inside the gate/up launch (pair indices kept as
// 16-bit entries of a 16 KB LDS list); larger calls run moe_route first.
constexpr int kRouteList = 8192;

// In-kernel routing of one expert (all threads of the workgroup call it):
// pairs are ranked in pair order, so the expert's pair indices land in
// plist[0, count) and its slots are begin .. begin + count - 1, with begin the
// number of valid pairs of lower expert ids (the segments of moe_route, which
// ranks inside a segment by atomic order instead; every (token, expert)
// product is independent of its place in the segment). Part 0 of the expert
// writes the routing tables the down GEMM and the combine read. Returns
// (begin, begin + count).
template <int W>
__device__ int2 route_expert(const Q4Tiled& p, int expert, bool writer, unsigned short* plist, int* rsum, int tid,
                             int lane, int wave) {
    constexpr int T = W * 64, PER = 8;
    int ranked = 0, below = 0, invalid = 0;
    for (int base = 0; base < p.pairs; base += T * PER) {
        const int i0 = base + PER * tid;
        std::int64_t e[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) e[u] = p.ids[min(i0 + u, p.pairs - 1)];
        int mine = 0, lo = 0, bad = 0;
        unsigned bits = 0;
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            if (i0 + u >= p.pairs) break;
            const bool ok = e[u] >= 0 && e[u] < p.experts;
            bad += !ok;
            lo += ok && e[u] < expert;
            if (e[u] == expert) {
                bits |= 1u << u;
                ++mine;
            }
            if (!ok && writer && expert == 0) p.pair_slot[i0 + u] = -1;
        }
        int incl = mine;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int other = __shfl_up(incl, d, 64);
            if (lane >= d) incl += other;
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            lo += __shfl_xor(lo, d, 64);
            bad += __shfl_xor(bad, d, 64);
        }
        if (lane == 63) rsum[wave] = incl;
        if (lane == 0) {
            rsum[W + wave] = lo;
            rsum[2 * W + wave] = bad;
        }
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const int c = rsum[w];
            before += w < wave ? c : 0;
            total += c;
            below += rsum[W + w];
            invalid += rsum[2 * W + w];
        }
        int rank = ranked + before + incl - mine;
#pragma unroll
        for (int u = 0; u < PER; ++u)
            if ((bits >> u) & 1u) plist[rank++] = static_cast<unsigned short>(i0 + u);
        ranked += total;
        __syncthreads();  // rsum is reused by the next batch; plist is whole after the last
    }
    if (writer) {
        if (tid == 0) {
            p.seg_out[expert + 1] = below + ranked;
            if (expert == 0) {
                p.seg_out[0] = 0;
                *p.status = invalid;
            }
        }
        for (int r = tid; r < ranked; r += T) {
            const int i = plist[r], slot = below + r;
            p.pair_slot[i] = slot;
            p.slot_token[slot] = i / p.top_k;
            p.slot_score[slot] = p.scores[i];
        }
    }
    return make_int2(below, below + ranked);
}

// Grouped expert GEMM over the tiled planes with a fraction of an expert per
// workgroup: W = 8 waves, wave v owns RB consecutive 16-row blocks (global
// block b = tile * 8 + w of the tiled layout), so a row tile (part) is 8 * RB
// blocks, whose activation chunks are staged once in LDS for all of them.
// Weights are double-buffered in registers by half chunk (1 KB per block):
// the loads of the next half are issued as soon as a half has been
// multiplied, so each wave keeps RB KB in flight. Each activation fragment is
// read from LDS once per step and multiplied by all RB blocks. Passes of up
// to 16 * NBMAX tokens.
//
// A workgroup carries TT consecutive row tiles of one expert. Under the last
// chunk of a tile the first chunk of the next (its weights and activations,
// into the same registers) is already in flight, so only the epilogue sits
// between two tiles, and the routing and the first chunk's latency (about
// 3-8 us per workgroup on MI355X at 128 experts x 512 tokens) are paid once.
// Down takes TT = 2: 128 experts x 8 tiles become 512 workgroups, two per
// CU, in one round instead of two (42 -> 35 us). Gate/up keeps TT = 1 (768
// workgroups filling the CUs as slots free): with TT = 2 its 384 workgroups
// leave half the CUs with two and half with one, and the CUs with two set the
// time; 512 workgroups of which a share carry two tiles measured no faster
// than one tile each (67.5 vs 67.3 us). TT = 1 compiles to the single-tile loop.
template <int EPI, int W, int RB, int NBMAX, bool ROUTE, int TT>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(4, 4))) void q4_grouped(Q4Tiled p, int parts,
                                                                                                int blocks) {
    __shared__ __attribute__((aligned(16))) _Float16 xl[2][16 * NBMAX * kXStride];
    __shared__ unsigned short plist[ROUTE ? kRouteList : 1];
    __shared__ int rsum[ROUTE ? 3 * W : 1];
    constexpr int kPass = 16 * NBMAX;

    const int linear = blockIdx.x;
    const int wgs = (parts + TT - 1) / TT;  // workgroups per expert
    int expert, wg;
    if (p.experts % 8 == 0) {  // an expert's workgroups share one XCD (round-robin dispatch) and its L2
        const int xcd = linear % 8, idx = linear / 8;
        expert = 8 * (idx / wgs) + xcd;
        wg = idx % wgs;
    } else {
        expert = linear / wgs;
        wg = linear % wgs;
    }
    const int first_part = wg * TT;
    const int tiles = min(TT, parts - first_part);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int seg_begin, seg_end;
    if constexpr (ROUTE) {
        const int2 range = route_expert<W>(p, expert, first_part == 0, plist, rsum, tid, lane, wave);
        seg_begin = range.x;
        seg_end = range.y;
    } else {
        seg_begin = p.seg[expert];
        seg_end = p.seg[expert + 1];
    }
    if (seg_begin >= seg_end) return;
    const int q = lane >> 4, m = lane & 15;
    constexpr int T = W * 64;
    // Unit offset of block r of tile t for this wave (wave-uniform); clamped
    // blocks are never stored.
    auto unit = [&](int t, int r) {
        const int b = min(((first_part + t) * W + wave) * RB + r, blocks - 1);
        return static_cast<std::int64_t>(b >> 3) * p.chunks * 8 + (b & 7);
    };
    std::int64_t unit0[RB];  // a single-tile workgroup's, computed once
#pragma unroll
    for (int r = 0; r < RB; ++r) unit0[r] = unit(0, r);
    const uint4* wbase = p.codes + expert * p.code_stride + lane;
    const __half* sbase = p.scales + expert * p.scale_stride + lane;

    for (int pass = seg_begin; pass < seg_end; pass += kPass) {
        const int live = min(kPass, seg_end - pass);
        auto run_pass = [&](auto nb_tag) {
            constexpr int NB = decltype(nb_tag)::value;
            // Activation staging: XL 16-byte pieces per thread cover the NB token
            // blocks (32 pieces per token row of a chunk).
            constexpr int XL = (NB * 512 + T - 1) / T;
            const __half* xrow[XL];
            bool xlive[XL];
#pragma unroll
            for (int j = 0; j < XL; ++j) {
                const int t = (tid + T * j) >> 5;
                xlive[j] = t < live && t < 16 * NB;
                const int slot = pass + min(t, live - 1);
                const int row = ROUTE ? plist[slot - seg_begin] / p.top_k : p.gather ? p.gather[slot] : slot;
                xrow[j] = p.x + static_cast<std::int64_t>(row) * p.x_stride;
            }
            struct Half {
                uint4 w[RB];
                unsigned short s[RB];
            };
            struct XStage {
                uint4 v[XL];
            };
            // Half h of chunk c of tile t for every block: 16 code bytes and the group scale.
            auto load_half = [&](int t, int c, int h, Half& st) {
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    const std::int64_t u = (TT == 1 ? unit0[r] : unit(t, r)) + static_cast<std::int64_t>(c) * 8;
                    st.w[r] = stream_load(wbase + u * 128 + 64 * h);
                    if (h == 0) st.s[r] = stream_load(reinterpret_cast<const unsigned short*>(sbase + u * 64));
                }
            };
            auto load_x = [&](int c, XStage& x) {
                const int col = c * kChunk + 8 * (tid & 31);
#pragma unroll
                for (int j = 0; j < XL; ++j) x.v[j] = *reinterpret_cast<const uint4*>(xrow[j] + min(col, p.k - 8));
            };
            auto store_x = [&](int c, const XStage& x, _Float16* buf) {
                const int col = c * kChunk + 8 * (tid & 31);
#pragma unroll
                for (int j = 0; j < XL; ++j) {
                    const int piece = tid + T * j;
                    const std::uint32_t keep = (xlive[j] && col < p.k) ? 0xFFFFFFFFu : 0u;
                    uint4 v = interleave_biased(x.v[j]);
                    v.x &= keep;
                    v.y &= keep;
                    v.z &= keep;
                    v.w &= keep;
                    if (NB * 512 % T == 0 || piece < NB * 512)  // rows past the pass's token blocks are not staged
                        *reinterpret_cast<uint4*>(buf + (piece >> 5) * kXStride + 8 * (piece & 31)) = v;
                }
            };

            float4v acc[RB][NB];

            // Multiplies half h of the current chunk (code words 4h .. 4h + 3 of
            // every block, activation columns 64q + 32h ..) from LDS buffer buf.
            unsigned short scale[RB];
            auto compute_half = [&](const Half& st, int h, const _Float16* buf) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    half8 xf[NB];
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        xf[b] = *reinterpret_cast<const half8*>(buf + (16 * b + m) * kXStride + 64 * q + 32 * h + 8 * s);
#pragma unroll
                    for (int r = 0; r < RB; ++r) {
                        const std::uint32_t word = s == 0 ? st.w[r].x : s == 1 ? st.w[r].y : s == 2 ? st.w[r].z : st.w[r].w;
                        const half2v s2 = __builtin_bit_cast(half2v, static_cast<std::uint32_t>(scale[r]) * 0x10001u);
                        const half8 wf = dequant8_biased(word, s2);
#pragma unroll
                        for (int b = 0; b < NB; ++b)
                            acc[r][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[b], wf, acc[r][b], 0, 0, 0);
                    }
                }
            };

            Half h0, h1;
            load_half(0, 0, 0, h0);
            load_half(0, 0, 1, h1);
            XStage xs;
            load_x(0, xs);
            store_x(0, xs, xl[0]);
            __syncthreads();
            for (int ti = 0; ti < tiles; ++ti) {
#pragma unroll
                for (int r = 0; r < RB; ++r)
#pragma unroll
                    for (int b = 0; b < NB; ++b) acc[r][b] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
                const bool more = ti + 1 < tiles;  // the next tile's first chunk follows this tile's last
                if constexpr (TT == 1) {
                    for (int c = 0; c < p.chunks; ++c) {
                        const int next = min(c + 1, p.chunks - 1);  // the last chunk re-reads itself (unused)
                        load_x(next, xs);
                        const _Float16* buf = xl[c & 1];
#pragma unroll
                        for (int r = 0; r < RB; ++r) scale[r] = h0.s[r];
                        compute_half(h0, 0, buf);
                        load_half(0, next, 0, h0);
                        compute_half(h1, 1, buf);
                        load_half(0, next, 1, h1);
                        store_x(c + 1, xs, xl[(c + 1) & 1]);
                        __syncthreads();
                    }
                } else {
                    for (int c = 0; c < p.chunks; ++c) {
                        const bool last = c + 1 == p.chunks;
                        // Next (tile, chunk): the following chunk, the next tile's first, or
                        // past the last tile's last chunk a re-read of it (unused).
                        const int nt = last && more ? ti + 1 : ti;
                        const int nc = last ? (more ? 0 : c) : c + 1;
                        load_x(nc, xs);
                        const _Float16* buf = xl[c & 1];
#pragma unroll
                        for (int r = 0; r < RB; ++r) scale[r] = h0.s[r];
                        compute_half(h0, 0, buf);
                        load_half(nt, nc, 0, h0);
                        compute_half(h1, 1, buf);
                        load_half(nt, nc, 1, h1);
                        if (!(last && more)) store_x(c + 1, xs, xl[(c + 1) & 1]);  // the next tile's chunk 0 waits for the epilogue
                        __syncthreads();
                    }
                }

                // Epilogue through LDS: the staging buffers are free after the last
                // chunk's barrier. The pass's output tile (tokens x the workgroup's
                // 16 W RB rows, or its 8 W RB SwiGLU columns) is written there from
                // the D layout (lane holds row slot m of block b for tokens
                // 16j + 4q + i), then every token row leaves as 16-byte stores: 2-byte
                // stores straight from the D layout leave 32-byte pieces of lines
                // that other workgroups also write (about 12 us of a 50 us launch at
                // 128 experts x 512 tokens x top-8). Row stride: 8 halves past the
                // tile width, so the four token quads of a store land on distinct
                // banks.
                constexpr int kOutCols = EPI == kSwiGLU ? W * RB * 8 : W * RB * 16;
                constexpr int kOutStride = kOutCols + 8;
                static_assert(16 * NBMAX * kOutStride <= 2 * 16 * NBMAX * kXStride, "the output tile fits the staging buffers");
                static_assert(W * RB % 8 == 0, "a workgroup covers whole SwiGLU column tiles");
                __half* tile = reinterpret_cast<__half*>(&xl[0][0]);
                const int first = (first_part + ti) * W * RB;  // the tile's first row block
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    const int slot_blk = wave * RB + r;
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int t = 16 * b + 4 * q + i;
                            const float v = acc[r][b][i];
                            if (EPI == kSwiGLU) {
                                const float other = __shfl_xor(v, 8, 64);  // lane m^8 holds the paired up/gate row
                                if (m < 8) {
                                    const float g = __half2float(from_f32<__half>(v));
                                    const float u = __half2float(from_f32<__half>(other));
                                    const float a = __half2float(from_f32<__half>(silu(g)));
                                    tile[t * kOutStride + 8 * slot_blk + m] = from_f32<__half>(__fmul_rn(a, u));
                                }
                            } else {
                                tile[t * kOutStride + 16 * slot_blk + m] = from_f32<__half>(v);  // scaled when stored
                            }
                        }
                    }
                }
                __syncthreads();
                // Rows t < live; columns of blocks past the last one, or past the
                // matrix, are not stored (SwiGLU columns of block blk start at
                // (blk >> 3) * 64 + 8 * (blk & 7); W * RB is a multiple of 8). The
                // column limit is a multiple of 8 (hidden and intermediate sizes
                // are), so a 16-byte unit is stored whole or not at all.
                const int col0 = EPI == kSwiGLU ? (first >> 3) * (kRows / 2) : 16 * first;
                const int limit = EPI == kSwiGLU ? p.half_rows : p.n;
                constexpr int kUnits = kOutCols / 8;
                for (int u = tid; u < live * kUnits; u += T) {
                    const int row = u / kUnits, c = 8 * (u % kUnits);
                    if (col0 + c < limit) {
                        uint4 w = *reinterpret_cast<const uint4*>(tile + row * kOutStride + c);
                        // fp16(fp16(y) * score), the product in fp32: applied here, one score per
                        // stored row unit, rather than per D-layout value, where the next tile's
                        // chunk is live in registers (twelve score loads per lane there spilled).
                        if constexpr (EPI == kScore) {
                            const float sc = __half2float(p.score[pass + row]);
                            std::uint32_t* h = reinterpret_cast<std::uint32_t*>(&w);
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const __half lo = from_f32<__half>(__fmul_rn(half_lo(h[j]), sc));
                                const __half hi = from_f32<__half>(__fmul_rn(half_hi(h[j]), sc));
                                h[j] = static_cast<std::uint32_t>(__half_as_ushort(lo)) |
                                       (static_cast<std::uint32_t>(__half_as_ushort(hi)) << 16);
                            }
                        }
                        *reinterpret_cast<uint4*>(p.out + static_cast<std::int64_t>(pass + row) * p.out_stride + col0 + c) = w;
                    }
                }
                if (more) {  // the staging buffers again hold activations: the next tile's first chunk
                    __syncthreads();
                    store_x(0, xs, xl[0]);
                    __syncthreads();
                }
            }
        };
        switch ((live + 15) >> 4) {
            case 1: run_pass(std::integral_constant<int, 1>{}); break;
            case 2: run_pass(std::integral_constant<int, (NBMAX >= 2 ? 2 : NBMAX)>{}); break;
            case 3: run_pass(std::integral_constant<int, (NBMAX >= 3 ? 3 : NBMAX)>{}); break;
            default: run_pass(std::integral_constant<int, NBMAX>{}); break;
        }
        __syncthreads();  // the next pass restages LDS
    }
}

// Routing: one workgroup of kRouteThreads. Pair i = token * top_k + position.
// Pass 1 counts pairs per expert (LDS atomics give each pair a rank in its
// expert); wave 0 turns the counts into segment offsets (each lane sums a run
// of experts, then a shuffle scan across the wave), and pass 2 places every
// pair at offset + rank. A batch is kRouteBatch pairs per thread, loaded up
// front; the first batch keeps its ids, scores and ranks in registers, later
// batches (more than kRouteThreads * kRouteBatch pairs) park their ranks in
// pair_slot between the passes. Three barriers for one batch.
constexpr int kRouteThreads = 512;
constexpr int kRouteBatch = 8;

__global__ __launch_bounds__(kRouteThreads) void moe_route(const std::int64_t* __restrict__ ids,
                                                           const __half* __restrict__ scores, int pairs, int top_k,
                                                           int experts, int* __restrict__ seg,
                                                           int* __restrict__ status, int* __restrict__ pair_slot,
                                                           int* __restrict__ slot_token,
                                                           __half* __restrict__ slot_score) {
    constexpr int T = kRouteThreads, B = kRouteBatch;
    __shared__ int count[kMaxExperts];
    __shared__ int base_of[kMaxExperts];
    __shared__ int invalid;
    const int tid = threadIdx.x;
    // The first batch's ids and scores are requested before the counters are cleared.
    std::int64_t first_e[B];
    __half first_sc[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
        const int i = min(u * T + tid, pairs - 1);
        first_e[u] = ids[i];
        first_sc[u] = scores[i];
    }
    for (int e = tid; e < experts; e += T) count[e] = 0;
    if (tid == 0) invalid = 0;
    __syncthreads();
    int first_rank[B];
    for (int base = 0; base < pairs; base += T * B) {
        std::int64_t e[B];
#pragma unroll
        for (int u = 0; u < B; ++u) e[u] = base == 0 ? first_e[u] : ids[min(base + u * T + tid, pairs - 1)];
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int i = base + u * T + tid;
            int rank = -1;
            if (i < pairs) {
                if (e[u] < 0 || e[u] >= experts) atomicAdd(&invalid, 1);
                else rank = atomicAdd(&count[e[u]], 1);
                if (base > 0) pair_slot[i] = rank;
            }
            if (base == 0) first_rank[u] = rank;
        }
    }
    __syncthreads();
    if (tid < 64) {
        const int run = (experts + 63) / 64;
        const int lo = min(tid * run, experts), hi = min(lo + run, experts);
        int own = 0;
        for (int e = lo; e < hi; ++e) own += count[e];
        int inclusive = own;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int other = __shfl_up(inclusive, d, 64);
            if (tid >= d) inclusive += other;
        }
        int offset = inclusive - own;
        for (int e = lo; e < hi; ++e) {
            base_of[e] = offset;
            offset += count[e];
            seg[e + 1] = offset;
        }
        if (tid == 0) {
            seg[0] = 0;
            *status = invalid;
        }
    }
    __syncthreads();
    for (int base = 0; base < pairs; base += T * B) {
        int rank[B];
        std::int64_t e[B];
        __half sc[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int i = min(base + u * T + tid, pairs - 1);
            rank[u] = base == 0 ? first_rank[u] : pair_slot[i];
            e[u] = base == 0 ? first_e[u] : ids[i];
            sc[u] = base == 0 ? first_sc[u] : scores[i];
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int i = base + u * T + tid;
            if (i < pairs) {
                int slot = -1;
                if (rank[u] >= 0) {
                    slot = base_of[e[u]] + rank[u];
                    slot_token[slot] = i / top_k;
                    slot_score[slot] = sc[u];
                }
                pair_slot[i] = slot;
            }
        }
    }
}

// Combine: one wave per token (4 tokens per 256-thread workgroup); each lane
// owns 8 consecutive columns per 512-column step. The token's slots are
// ordered by ascending expert id (stable: position order for repeated ids) and
// added in that order from +0 with fp16 adds, as index_add_ does per expert.
// A token with an expert id outside [0, experts) (the reference rejects such
// routing) gets a NaN row, so the error shows without a host synchronisation.
template <int K>
__global__ __launch_bounds__(256) void moe_combine(const std::int64_t* __restrict__ ids,
                                                   const int* __restrict__ pair_slot, const __half* __restrict__ v,
                                                   __half* __restrict__ out, int tokens, int hidden) {
    // One 4-wave workgroup per token, each wave a quarter of the columns (every
    // wave sorts the token's K pairs itself).
    const int token = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int order[K];
    std::int64_t key[K];
    int n = 0;
#pragma unroll
    for (int p = 0; p < K; ++p) {
        order[p] = pair_slot[token * K + p];
        key[p] = order[p] < 0 ? INT64_MAX : ids[token * K + p];  // skipped pairs sort last
        n += order[p] >= 0;
    }
    // Stable bubble sort with static indices (keeps the arrays in registers).
#pragma unroll
    for (int i = 0; i < K; ++i)
#pragma unroll
        for (int j = 0; j + 1 < K - i; ++j)
            if (key[j] > key[j + 1]) {
                const std::int64_t tk = key[j];
                key[j] = key[j + 1];
                key[j + 1] = tk;
                const int to = order[j];
                order[j] = order[j + 1];
                order[j + 1] = to;
            }
    for (int col = 8 * lane + 512 * wave; col < hidden; col += 4 * 512) {
        uint4 r[K];
#pragma unroll
        for (int i = 0; i < K; ++i)
            r[i] = *reinterpret_cast<const uint4*>(v + static_cast<std::int64_t>(max(order[i], 0)) * hidden + col);
        half2v acc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = half2v{static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f)};
#pragma unroll
        for (int i = 0; i < K; ++i) {
            if (i < n) {
                acc[0] += __builtin_bit_cast(half2v, r[i].x);
                acc[1] += __builtin_bit_cast(half2v, r[i].y);
                acc[2] += __builtin_bit_cast(half2v, r[i].z);
                acc[3] += __builtin_bit_cast(half2v, r[i].w);
            }
        }
        uint4 o;
        o.x = __builtin_bit_cast(std::uint32_t, acc[0]);
        o.y = __builtin_bit_cast(std::uint32_t, acc[1]);
        o.z = __builtin_bit_cast(std::uint32_t, acc[2]);
        o.w = __builtin_bit_cast(std::uint32_t, acc[3]);
        if (n < K) o = make_uint4(0x7e007e00u, 0x7e007e00u, 0x7e007e00u, 0x7e007e00u);  // fp16 quiet NaNs
        *reinterpret_cast<uint4*>(out + static_cast<std::int64_t>(token) * hidden + col) = o;
    }
}

template <int K>
void launch_combine(const std::int64_t* ids, const int* pair_slot, const __half* v, __half* out, int tokens,
                    int hidden, hipStream_t stream) {
    moe_combine<K><<<tokens, 256, 0, stream>>>(ids, pair_slot, v, out, tokens, hidden);
}

void combine_dispatch(int top_k, const std::int64_t* ids, const int* pair_slot, const __half* v, __half* out,
                      int tokens, int hidden, hipStream_t stream) {
    switch (top_k) {
#define VT_CASE(K) \
    case K: launch_combine<K>(ids, pair_slot, v, out, tokens, hidden, stream); break;
        VT_CASE(1) VT_CASE(2) VT_CASE(3) VT_CASE(4) VT_CASE(5) VT_CASE(6) VT_CASE(7) VT_CASE(8)
        VT_CASE(9) VT_CASE(10) VT_CASE(11) VT_CASE(12) VT_CASE(13) VT_CASE(14) VT_CASE(15) VT_CASE(16)
#undef VT_CASE
        default: throw Invalid("top_k must be in [1, 16]");
    }
}

template <int EPI, int W, int RB, int NBMAX, bool ROUTE, int TT>
void launch_q4_grouped(const Q4Tiled& p, hipStream_t stream) {
    const int blocks = p.row_tiles * 8;
    const int parts = (blocks + W * RB - 1) / (W * RB);
    const int wgs = (parts + TT - 1) / TT;
    q4_grouped<EPI, W, RB, NBMAX, ROUTE, TT><<<dim3(p.experts * wgs), W * 64, 0, stream>>>(p, parts, blocks);
}

std::uint64_t align256(std::uint64_t v) { return (v + 255) / 256 * 256; }

// ---------------------------------------------------------------------------
// W4/5/6A16 prefill GEMM (many tokens): out[t][n] = fp16(sum_k x[t][k] * w[n][k])
// with the contract weights w = fp16(q * scale) (one rounding each, as the
// reference's fp16 shadow). Once the weights are fp16 the product is a plain
// fp16 GEMM: the matrix cores accumulate across groups and no per-group VALU
// work remains. A workgroup of WM x WN waves computes (WM*TI*16) tokens x
// (WN*TJ*16) rows; one 64-column group per stage: the tile's activation rows
// (64 halves, staged in dequant8's column order) and weight rows (dequantized
// once per workgroup into fp16) in two LDS buffers. Rows are eight 16-byte
// units XOR-swizzled by (row >> 1) & 7, so 16 consecutive rows' fragment reads
// cover all 64 banks once. Global loads run PF groups ahead in registers.
template <int WM, int WN, int TI, int TJ, int GS>
struct RowPrefillGeom {
    static constexpr int kThreads = WM * WN * 64;
    static constexpr int kTM = WM * TI * 16;
    static constexpr int kTN = WN * TJ * 16;
    static constexpr int kU = 8 * GS;             // 16-byte units of a staged row (64 halves a group)
    static constexpr int kAUnits = kTM * kU;      // 16-byte activation loads per stage
    static constexpr int kBUnits = kTN * 2 * GS;  // 16-byte code loads per stage (32 code bytes a row a group)
    static constexpr int kAPer = (kAUnits + kThreads - 1) / kThreads;
    static constexpr int kBPer = (kBUnits + kThreads - 1) / kThreads;
    static constexpr std::size_t kLds = 2 * static_cast<std::size_t>(kTM + kTN) * kU * 16;
    static_assert(kAUnits % kThreads == 0, "whole activation loads per thread");
    static_assert(kLds <= 160 * 1024, "prefill tiles exceed LDS");
};

__device__ __forceinline__ int swizzle8(int row) { return (row >> 1) & 7; }

// GS groups (64 columns each) per stage, one barrier per stage; a staged row
// holds the stage's groups one after another, each group's eight units
// swizzled as above.
template <int HB, int WM, int WN, int TI, int TJ, int PF, int GS>
__global__ __launch_bounds__(WM * WN * 64) void row_prefill(const __half* __restrict__ x,
                                                           const std::uint8_t* __restrict__ codes,
                                                           const std::uint8_t* __restrict__ high,
                                                           const __half* __restrict__ scales, __half* __restrict__ out,
                                                           int tokens, int n, int k, int padded) {
    using G = RowPrefillGeom<WM, WN, TI, TJ, GS>;
    constexpr int TM = G::kTM, TN = G::kTN, T = G::kThreads, U = G::kU;
    struct Stage {
        uint4 a[G::kAPer];
        uint4 b[G::kBPer];
        std::uint32_t h[G::kBPer][HB ? HB : 1];
        unsigned short s[G::kBPer];
    };
    // Dynamic LDS: two activation buffers [TM * U], then two weight buffers [TN * U].
    extern __shared__ uint4 rp_lds[];
    auto* a_lds = reinterpret_cast<uint4(*)[TM * U]>(rp_lds);
    auto* b_lds = reinterpret_cast<uint4(*)[TN * U]>(rp_lds + 2 * TM * U);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int q = lane >> 4, r = lane & 15;
    const int t0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
    const int groups = padded / 64;
    const int stages = (groups + GS - 1) / GS;

    // Activation unit i = tid + u*T: token i / U, group (i / 8) % GS of the
    // stage, columns 8 * (i % 8) of that group.
    const __half* a_src[G::kAPer];
    bool a_row_ok[G::kAPer];
#pragma unroll
    for (int u = 0; u < G::kAPer; ++u) {
        const int tok = (tid + u * T) / U;
        a_row_ok[u] = t0 + tok < tokens;
        a_src[u] = x + static_cast<std::int64_t>(min(t0 + tok, tokens - 1)) * k;
    }
    // Code unit i: row i / (2 GS), group (i / 2) % GS of the stage, code bytes
    // 16 * (i % 2) of that group (columns 32 * (i % 2) ..).
    std::int64_t b_row[G::kBPer];
#pragma unroll
    for (int u = 0; u < G::kBPer; ++u) b_row[u] = min(n0 + min((tid + u * T) / (2 * GS), TN - 1), n - 1);

    // Groups past the last one (groups % GS != 0) are read clamped to the last
    // group; their activations are stored as zeros.
    auto load = [&](int sg, Stage& st) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < G::kAPer; ++u) {
            const int i = tid + u * T;
            const int g = sg * GS + (i / 8) % GS;
            st.a[u] = *reinterpret_cast<const uint4*>(a_src[u] + min(64 * g + 8 * (i & 7), k - 8));
        }
#pragma unroll
        for (int u = 0; u < G::kBPer; ++u) {
            const int i = tid + u * T;
            if (G::kBUnits % T != 0 && i >= G::kBUnits) break;
            const int half = i & 1;
            const int g = min(sg * GS + (i / 2) % GS, groups - 1);
            st.b[u] = *reinterpret_cast<const uint4*>(codes + b_row[u] * (padded / 2) + 32 * g + 16 * half);
            st.s[u] = __half_as_ushort(scales[b_row[u] * groups + g]);
            if constexpr (HB > 0) {
                // 32 columns x HB bits = 4 * HB bytes of the row's high stream.
                const std::uint8_t* hp = high + b_row[u] * (padded * HB / 8) + (64 * g + 32 * half) * HB / 8;
#pragma unroll
                for (int w = 0; w < HB; ++w) st.h[u][w] = reinterpret_cast<const std::uint32_t*>(hp)[w];
            }
        }
    };
    auto store = [&](const Stage& st, int sg, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < G::kAPer; ++u) {
            const int i = tid + u * T;
            const int tok = i / U, gg = (i / 8) % GS, unit = i & 7;
            const bool ok = a_row_ok[u] && 64 * (sg * GS + gg) + 8 * unit < k;  // k % 8 == 0: a unit is all in or all out
            a_lds[buf][tok * U + gg * 8 + (unit ^ swizzle8(tok))] = ok ? interleave8(st.a[u]) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < G::kBPer; ++u) {
            const int i = tid + u * T;
            if (G::kBUnits % T != 0 && i >= G::kBUnits) break;
            const int row = i / (2 * GS), gg = (i / 2) % GS, half = i & 1;
            const half2v s2 = __builtin_bit_cast(half2v, static_cast<std::uint32_t>(st.s[u]) * 0x10001u);
            const std::uint32_t words[4] = {st.b[u].x, st.b[u].y, st.b[u].z, st.b[u].w};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                half8 v;
                if constexpr (HB == 0) {
                    v = dequant8(words[w], s2);
                } else {
                    // Word w covers 8 columns: bits 8 * HB * w .. of the 32 * HB loaded.
                    const std::uint32_t hbits = (st.h[u][(HB * w) >> 2] >> (8 * ((HB * w) & 3))) & ((1u << (8 * HB)) - 1u);
                    v = dequant8_high<HB>(words[w], hbits, s2);
                }
                b_lds[buf][row * U + gg * 8 + ((4 * half + w) ^ swizzle8(row))] = __builtin_bit_cast(uint4, v);
            }
        }
    };

    float4v acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int gg = 0; gg < GS; ++gg)
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) {  // two 32-column slices of the group
            half8 fb[TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int row = wn * TJ * 16 + j * 16 + r;
                fb[j] = __builtin_bit_cast(half8, b_lds[buf][row * U + gg * 8 + ((4 * sl + q) ^ swizzle8(row))]);
            }
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const int tok = wm * TI * 16 + i * 16 + r;
                const half8 fa = __builtin_bit_cast(half8, a_lds[buf][tok * U + gg * 8 + ((4 * sl + q) ^ swizzle8(tok))]);
#pragma unroll
                for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa, fb[j], acc[i][j], 0, 0, 0);
            }
        }
    };

    Stage st[PF];
#pragma unroll
    for (int s = 0; s < PF; ++s) load(min(s, stages - 1), st[s]);
    store(st[0], 0, 0);
    if (PF < stages) load(PF, st[0]);
    __syncthreads();
    for (int g0 = 0; g0 < stages; g0 += PF) {
#pragma unroll
        for (int s = 0; s < PF; ++s) {
            const int g = g0 + s;
            if (g >= stages) break;
            compute(g & 1);
            if (g + 1 < stages) {
                store(st[(s + 1) % PF], g + 1, (g + 1) & 1);
                if (g + 1 + PF < stages) load(g + 1 + PF, st[(s + 1) % PF]);
            }
            __syncthreads();
        }
    }

#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int row = n0 + wn * TJ * 16 + j * 16 + r;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = t0 + wm * TI * 16 + i * 16 + 4 * q + e;
                if (t < tokens && row < n) out[static_cast<std::int64_t>(t) * n + row] = from_f32<__half>(acc[i][j][e]);
            }
        }
}

template <int HB, int WM, int WN, int TI, int TJ, int PF, int GS = 1>
void launch_row_prefill(const __half* x, const std::uint8_t* codes, const std::uint8_t* high, const __half* scales,
                        __half* out, int tokens, int n, int k, int padded, hipStream_t stream) {
    using G = RowPrefillGeom<WM, WN, TI, TJ, GS>;
    const dim3 grid((n + G::kTN - 1) / G::kTN, (tokens + G::kTM - 1) / G::kTM);
    require(grid.y <= 65535, "token tiles exceed the launch grid");
    if constexpr (G::kLds > 64 * 1024) {
        static const hipError_t raised = hipFuncSetAttribute(
            reinterpret_cast<const void*>(row_prefill<HB, WM, WN, TI, TJ, PF, GS>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(G::kLds));
        check(raised);
    }
    row_prefill<HB, WM, WN, TI, TJ, PF, GS><<<grid, G::kThreads, G::kLds, stream>>>(x, codes, high, scales, out,
                                                                                   tokens, n, k, padded);
}

// ---------------------------------------------------------------------------
// W4/5/6A16 decode GEMM (fewer tokens than the prefill tiles) over the
// row-major planes: out[t][n] = fp16(sum_k x[t][k] * fp16(q * scale)), fp32
// accumulation. A workgroup of W waves owns RB blocks of 16 weight rows and its
// waves split the K range; a lane (r, q) of a wave reads, per 128-column chunk,
// the 16 code bytes of row r holding columns 32q .. 32q+31 (a row block's chunk
// is one 1 KB wave load of 64-byte row segments), the pair of group scales of
// the chunk and, for Q5/Q6, the 4 * HB high-plane bytes of those columns. The
// four code words become four half8 B fragments (dequant8 order) for four
// v_mfma_f32_16x16x32_f16 whose A fragments are the matching activations of
// token r (interleave8); lanes of absent tokens load the last token's row and
// feed output rows that are never stored. Chunks are
// fetched in a two-deep ping-pong; partial tiles are summed across waves
// through LDS in wave order and stored by one wave per (row block, token block).
//
// TILED reads the decode copy built by q4.tile_q4 / q5.tile_row_codec instead: codes
// [row block][chunk][lane 16q + r][16 bytes] holding the code bytes lane (r, q)
// reads from the row-major planes, and scales [row block][chunk][r][2] (the
// chunk's two groups); each load is then one contiguous 1 KB (codes) or
// 64-byte (scales) wave access. The copy stores each word's nibbles pre-biased
// (q + 8) and reordered (nibble j holds column 2j, nibble 4 + j column 2j + 1)
// so that dequant8_biased yields the eight columns in natural order: the
// activation fragments need no interleave. Q5/Q6 copies order the nibbles the
// same way (unbiased) and tile the high plane [row block][chunk][lane][HB
// registers] with each column's upper bits biased (sign flipped) and placed so
// that dequant8_biased_high reads a column pair's fields with one shift and
// one mask-and-or (the layout is q5.tile_row_codec's). Every product and sum
// is the same as in the row-major path (the MFMA's k slots hold the same
// column pairs), so both layouts give the same bits.
template <int HB, int RB, int NB, int STEPS>
struct RowDecodeBatch {
    uint4 w[STEPS][RB];
    std::uint32_t s[STEPS][RB];
    std::uint32_t h[STEPS][RB][HB ? HB : 1];
    uint4 x[STEPS][NB][4];
};

// Idle pattern of a split-K exchange slot: two signalling NaNs, which no
// arithmetic result takes.
constexpr unsigned long long kRowSlotEmpty = 0x7f8000017f800001ull;

template <int HB, int W, int RB, int NB, int STEPS, bool TILED, int KS>
__global__ __launch_bounds__(W * 64) void row_decode_gemm(const __half* __restrict__ x,
                                                          const std::uint8_t* __restrict__ codes,
                                                          const std::uint8_t* __restrict__ high,
                                                          const __half* __restrict__ scales, __half* __restrict__ out,
                                                          unsigned long long* __restrict__ slots, int tokens, int n,
                                                          int k, int padded) {
    __shared__ float4v partial[W][RB * NB][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r = lane & 15;
    const int block0 = static_cast<int>(blockIdx.x / KS) * RB;
    const int chunks = padded / 128;
    // KS == 2: workgroups 2g and 2g + 1 take the first and second half of the
    // chunks of row-block group g; the W waves split that range evenly.
    const int kper = (chunks + KS - 1) / KS;
    const int k0 = KS == 1 ? 0 : min(static_cast<int>(blockIdx.x % KS) * kper, chunks);
    const int k1 = KS == 1 ? chunks : min(k0 + kper, chunks);
    const int c0 = k0 + wave * (k1 - k0) / W, c1 = k0 + (wave + 1) * (k1 - k0) / W;
    const std::int64_t cstride = padded / 2, sstride = padded / 64, hstride = padded * HB / 8;
    const std::uint8_t* cp[RB];
    const std::uint32_t* sp[RB];
    const std::uint8_t* hp[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        if constexpr (TILED) {
            const std::int64_t blk = min(block0 + b, (n + 15) / 16 - 1);  // clamped blocks are never stored
            cp[b] = codes + blk * chunks * 1024 + 16 * lane;
            sp[b] = reinterpret_cast<const std::uint32_t*>(scales) + blk * chunks * 16 + r;
            hp[b] = HB ? high + blk * chunks * 256 * HB + 4 * HB * lane : nullptr;
        } else {
            const std::int64_t row = min((block0 + b) * 16 + r, n - 1);  // clamped rows are never stored
            cp[b] = codes + row * cstride + 16 * q;
            sp[b] = reinterpret_cast<const std::uint32_t*>(scales + row * sstride);
            hp[b] = HB ? high + row * hstride + 4 * HB * q : nullptr;
        }
    }
    const __half* xr[NB];
#pragma unroll
    for (int tb = 0; tb < NB; ++tb)
        xr[tb] = x + static_cast<std::int64_t>(min(16 * tb + r, tokens - 1)) * k + 32 * q;
    const BiasedMasks masks = biased_masks();
    const HighMasks hmasks = TILED && HB > 0 ? high_masks<HB ? HB : 1>() : HighMasks{0u, 0u};
    using Batch = RowDecodeBatch<HB, RB, NB, STEPS>;
    const int batches = (c1 - c0 + STEPS - 1) / STEPS;
    // Batch i holds chunks c0 + i * STEPS + s; chunks past c1 are clamped to c1 - 1
    // when loaded and skipped when multiplied.
    auto fetch = [&](int i, Batch& t) __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
            const int c = min(c0 + i * STEPS + st, c1 - 1);
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                t.w[st][b] = stream_load(reinterpret_cast<const uint4*>(cp[b] + (TILED ? 1024 : 64) * c));
                t.s[st][b] = stream_load(sp[b] + (TILED ? 16 * c : c));
                if constexpr (HB > 0) {
#pragma unroll
                    for (int h = 0; h < HB; ++h)
                        t.h[st][b][h] =
                            reinterpret_cast<const std::uint32_t*>(hp[b] + (TILED ? 256 * HB : 16 * HB) * c)[h];
                }
            }
            // A chunk wholly inside k loads every lane's fragments unmasked: lanes of
            // absent tokens read the last token's row (valid memory) and feed only
            // output rows that are never stored. The chunk that crosses k
            // (k % 128 != 0) zeroes columns at or past k (k % 8 == 0: a fragment is
            // all in or all out).
            const int col = 128 * c + 32 * q;
            if (128 * c + 128 <= k) {
#pragma unroll
                for (int tb = 0; tb < NB; ++tb)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        t.x[st][tb][j] = *reinterpret_cast<const uint4*>(xr[tb] + 128 * c + 8 * j);
            } else {
#pragma unroll
                for (int tb = 0; tb < NB; ++tb)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        uint4 v = make_uint4(0u, 0u, 0u, 0u);
                        if (col + 8 * j < k) v = *reinterpret_cast<const uint4*>(xr[tb] + 128 * c + 8 * j);
                        t.x[st][tb][j] = v;
                    }
            }
        }
    };
    float4v acc[RB][NB];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int tb = 0; tb < NB; ++tb) acc[b][tb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    auto consume = [&](int i, const Batch& t) __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < STEPS; ++st) {
        if (c0 + i * STEPS + st >= c1) break;
        half8 fa[NB][4];
#pragma unroll
        for (int tb = 0; tb < NB; ++tb)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                fa[tb][j] = __builtin_bit_cast(half8, TILED ? t.x[st][tb][j] : interleave8(t.x[st][tb][j]));
#pragma unroll
        for (int b = 0; b < RB; ++b) {
            // Columns 32q .. 32q+31 of the chunk lie in its group q / 2.
            const std::uint32_t s = (t.s[st][b] >> (16 * (q >> 1))) & 0xFFFFu;
            const half2v s2 = __builtin_bit_cast(half2v, s * 0x10001u);
            const std::uint32_t words[4] = {t.w[st][b].x, t.w[st][b].y, t.w[st][b].z, t.w[st][b].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                half8 wf;
                if constexpr (TILED && HB == 0) {
                    wf = dequant8_biased(words[j], s2, masks);
                } else if constexpr (TILED) {
                    wf = dequant8_biased_high<HB>(words[j], t.h[st][b][(HB * j) >> 2], j % (4 / HB), s2, masks,
                                                  hmasks);
                } else if constexpr (HB == 0) {
                    wf = dequant8(words[j], s2);
                } else {
                    // Word j's eight columns own bits 8 * HB * j .. of the lane's 32 * HB.
                    const std::uint32_t hbits =
                        (t.h[st][b][(HB * j) >> 2] >> (8 * ((HB * j) & 3))) & ((1u << (8 * HB)) - 1u);
                    wf = dequant8_high<HB>(words[j], hbits, s2);
                }
#pragma unroll
                for (int tb = 0; tb < NB; ++tb)
                    acc[b][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[tb][j], wf, acc[b][tb], 0, 0, 0);
            }
        }
        }
    };
    if (batches > 0) {
        Batch ta, tb2;
        fetch(0, ta);
        for (int i = 0; i < batches; i += 2) {
            if (i + 1 < batches) fetch(i + 1, tb2);
            consume(i, ta);
            if (i + 1 >= batches) break;
            if (i + 2 < batches) fetch(i + 2, ta);
            consume(i + 1, tb2);
        }
    }
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int tb = 0; tb < NB; ++tb) partial[wave][b * NB + tb][lane] = acc[b][tb];
    __syncthreads();
    for (int p = wave; p < RB * NB; p += W) {
        const int b = p / NB, tb = p % NB;
        float4v sum = partial[0][p][lane];
        for (int w = 1; w < W; ++w) {
            const float4v v = partial[w][p][lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) sum[e] += v[e];
        }
        // D layout: lane (r, q) holds tokens 4q .. 4q+3 of the token block for weight row r.
        const int blk = block0 + b, row = blk * 16 + r;
        if constexpr (KS == 1) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = 16 * tb + 4 * q + e;
                if (t < tokens && row < n) out[static_cast<std::int64_t>(t) * n + row] = from_f32<__half>(sum[e]);
            }
        } else {
            // Pairwise exchange of the two K halves through a 64-bit slot per
            // (token, block, row pair r, r + 8): the first half leaves its pair, the
            // second adds (two fp32 terms: the result does not depend on the
            // arrival order), stores and returns the slot to idle. Only the slot is
            // shared, so no fence is needed, and every call leaves the slots idle.
            // All four exchanges of a lane are issued before any result is used
            // (one atomic round trip, not four in sequence).
            const int blocks = (n + 15) / 16;
            float partner[4];
            unsigned long long old[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) partner[e] = __shfl_xor(sum[e], 8, 64);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = 16 * tb + 4 * q + e;
                old[e] = kRowSlotEmpty;
                if (r < 8 && t < tokens && blk < blocks) {
                    unsigned long long* slot = slots + (static_cast<std::int64_t>(t) * blocks + blk) * 8 + r;
                    const unsigned long long packed =
                        (static_cast<unsigned long long>(__float_as_uint(partner[e])) << 32) | __float_as_uint(sum[e]);
                    old[e] = __hip_atomic_exchange(slot, packed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = 16 * tb + 4 * q + e;
                if (r < 8 && t < tokens && blk < blocks && old[e] != kRowSlotEmpty) {
                    unsigned long long* slot = slots + (static_cast<std::int64_t>(t) * blocks + blk) * 8 + r;
                    __hip_atomic_store(slot, kRowSlotEmpty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    const float lo = sum[e] + __uint_as_float(static_cast<std::uint32_t>(old[e]));
                    const float hi = partner[e] + __uint_as_float(static_cast<std::uint32_t>(old[e] >> 32));
                    __half* o = out + static_cast<std::int64_t>(t) * n;
                    if (row < n) o[row] = from_f32<__half>(lo);
                    if (row + 8 < n) o[row + 8] = from_f32<__half>(hi);
                }
            }
        }
    }
}

__global__ void fill_row_slots(unsigned long long* __restrict__ slots, std::size_t count) {
    for (std::size_t i = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; i < count;
         i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
        slots[i] = kRowSlotEmpty;
}

void fill_row_slot_buffer(unsigned long long* slots, std::size_t bytes, hipStream_t stream) {
    const std::size_t count = bytes / 8;
    if (count)
        fill_row_slots<<<static_cast<unsigned>(std::min<std::size_t>((count + 255) / 256, 1024)), 256, 0, stream>>>(
            slots, count);
}

// After a split decode's launch: a refused launch never ran and left the
// slots idle; they are refilled anyway (best effort) before the error is
// raised, so a caller never has to reason about their state.
void settle_row_slots(unsigned long long* slots, std::size_t bytes, hipStream_t stream) {
    const hipError_t launched = hipGetLastError();
    if (launched != hipSuccess) {
        if (slots) fill_row_slot_buffer(slots, bytes, stream);
        check(launched);
    }
}

template <int HB, int W, int RB, int NB, int STEPS, bool TILED, int KS = 1>
void launch_row_decode(const __half* x, const std::uint8_t* codes, const std::uint8_t* high, const __half* scales,
                       __half* out, int tokens, int n, int k, int padded, hipStream_t stream,
                       unsigned long long* slots = nullptr) {
    require(KS == 1 || slots, "a split decode needs its slot buffer");
    const int blocks = (n + 15) / 16;
    row_decode_gemm<HB, W, RB, NB, STEPS, TILED, KS><<<(blocks + RB - 1) / RB * KS, W * 64, 0, stream>>>(
        x, codes, high, scales, out, slots, tokens, n, k, padded);
}

}  // namespace

// Workspace of one MoE call (offsets in bytes, each section 256-byte aligned):
// seg int32[experts+1], status int32, pair_slot int32[P], slot_token int32[P],
// slot_score fp16[P], h fp16[P][inter], v fp16[P][hidden]; P = tokens * top_k.
struct MoELayout {
    std::uint64_t seg, status, pair_slot, slot_token, slot_score, h, v, total;
};

MoELayout moe_layout(std::int64_t tokens, std::int64_t top_k, std::int64_t experts, std::int64_t hidden,
                     std::int64_t inter) {
    const std::uint64_t pairs = static_cast<std::uint64_t>(tokens * top_k);
    MoELayout l;
    l.seg = 0;
    l.status = align256(4 * (experts + 1));
    l.pair_slot = l.status + 256;
    l.slot_token = l.pair_slot + align256(4 * pairs);
    l.slot_score = l.slot_token + align256(4 * pairs);
    l.h = l.slot_score + align256(2 * pairs);
    l.v = l.h + align256(2 * pairs * inter);
    l.total = l.v + align256(2 * pairs * hidden);
    return l;
}

void moe_validate(int tokens, int top_k, int experts, int hidden, int inter) {
    require(tokens > 0 && top_k > 0 && top_k <= 16 && experts > 0 && experts <= kMaxExperts,
            "MoE needs tokens > 0, 0 < top_k <= 16, 0 < experts <= 1024");
    require(hidden > 0 && inter > 0 && hidden % 8 == 0 && inter % 8 == 0,
            "MoE hidden and intermediate sizes must be positive multiples of 8");
    require(static_cast<std::int64_t>(tokens) * top_k * std::max(hidden, 2 * inter) < INT32_MAX,
            "MoE routed rows exceed int32 geometry");
}

// Decode launch shapes, measured at the config-2 matrices (QKV 448 row blocks,
// o_proj and down 320, gate+up 2176) at 1-24 tokens: 16 waves over two row
// blocks for up to 384 blocks, 8 waves over two up to 1023 and over three
// from 1024; two token blocks (17-31 tokens) take 8 waves over two.
// The tiled Q4 decode splits K over two workgroups (8 waves over 3 row blocks
// each, slots exchanged pairwise) for up to 384 row blocks with at least 64
// chunks of 128 columns: there the unsplit grid leaves most CUs with one long
// workgroup (down 17408 -> 5120: 16.4 -> 14.3 us at one token, 24.1 -> 18.8 at
// 16); with shorter K (o_proj, 48 chunks) the split measured no faster.
bool row_decode_splits(int tokens, int n, int padded) {
    return tokens <= 16 && (n + 15) / 16 <= 384 && padded / 128 >= 64;
}

std::uint64_t row_decode_slot_bytes(int tokens, int n, int padded) {
    return row_decode_splits(tokens, n, padded)
               ? static_cast<std::uint64_t>(tokens) * ((n + 15) / 16) * 8 * sizeof(unsigned long long)
               : 0;
}

template <int HB, bool TILED = false>
void row_decode_dispatch(const __half* x, const std::uint8_t* codes, const std::uint8_t* high, const __half* scales,
                         __half* out, int tokens, int n, int k, int padded, hipStream_t stream,
                         unsigned long long* slots = nullptr) {
    const int blocks = (n + 15) / 16;
    if (TILED && row_decode_splits(tokens, n, padded))
        launch_row_decode<HB, 8, 3, 1, 1, TILED, 2>(x, codes, high, scales, out, tokens, n, k, padded, stream, slots);
    else if (tokens > 16)
        launch_row_decode<HB, 8, 2, 2, 1, TILED>(x, codes, high, scales, out, tokens, n, k, padded, stream);
    else if (blocks <= 384)
        launch_row_decode<HB, 16, 2, 1, 1, TILED>(x, codes, high, scales, out, tokens, n, k, padded, stream);
    else if (blocks < 1024)
        launch_row_decode<HB, 8, 2, 1, 1, TILED>(x, codes, high, scales, out, tokens, n, k, padded, stream);
    else
        launch_row_decode<HB, 8, 3, 1, 1, TILED>(x, codes, high, scales, out, tokens, n, k, padded, stream);
}

// Token count from which the W4/5/6A16 GEMM uses the prefill tiles (128 tokens
// x 128 rows, which read each weight once per 128 tokens; below it the decode
// GEMM reads each weight once per 16 or 32 tokens).
constexpr int kRowPrefillMinTokens = 32;

// Prefill tiles. Below 256 tokens: 128 tokens x 128 rows (8 waves of 32 x 64).
// From 256 tokens: 256 tokens x 32*TJ rows, 8 waves of 64 x 16*TJ (one
// workgroup per CU by LDS), TJ in {5, 6, 7} picked for the fewest tile rounds
// over the CUs weighted by the wider tiles' higher rate (fewer LDS bytes per
// MFMA): at M = 2048 on MI355X, 5120 rows take TJ = 5 (256 tiles, one round),
// 7168 and 34816 rows TJ = 7 (config-2 W4A16 at M = 2048: QKV / o_proj /
// gate+up / down 214 / 196 / 908 / 532 -> 155-162 / 144-151 / 729-774 /
// 386-409 us against 128 x 128 tiles; same bytes).
template <int HB>
void row_prefill_dispatch(const __half* x, const std::uint8_t* codes, const std::uint8_t* high, const __half* scales,
                          __half* out, int tokens, int n, int k, int padded, hipStream_t stream) {
    if (tokens < 256) {
        launch_row_prefill<HB, 4, 2, 2, 4, 2>(x, codes, high, scales, out, tokens, n, k, padded, stream);
        return;
    }
    const int cus = device_cus();
    const std::int64_t token_tiles = (tokens + 255) / 256;
    int best = 5;
    double best_cost = 0.0;
    for (int tj = 5; tj <= 7; ++tj) {
        const std::int64_t tiles = token_tiles * ((n + 32 * tj - 1) / (32 * tj));
        const double rate = tj == 5 ? 1.0 : tj == 6 ? 1.1 : 1.2;  // work per unit time, measured
        const double cost = static_cast<double>((tiles + cus - 1) / cus) * tj / rate;
        if (tj == 5 || cost < best_cost) {
            best = tj;
            best_cost = cost;
        }
    }
    if (best == 5) launch_row_prefill<HB, 4, 2, 4, 5, 2>(x, codes, high, scales, out, tokens, n, k, padded, stream);
    else if (best == 6) launch_row_prefill<HB, 4, 2, 4, 6, 2>(x, codes, high, scales, out, tokens, n, k, padded, stream);
    else launch_row_prefill<HB, 4, 2, 4, 7, 1>(x, codes, high, scales, out, tokens, n, k, padded, stream);
}

void row_gemm_launch(const void* x, const void* codes, const void* high, const void* scales, void* out, int tokens,
                     int n, int k, int padded, int bits, int dtype, hipStream_t stream) {
    require(bits == 4 || bits == 5 || bits == 6, "row codecs are 4, 5 or 6 bits");
    require(x && codes && scales && out && (bits == 4 || high), "null Q4/Q5/Q6 operand");
    require(tokens > 0 && n > 0 && k > 0 && padded == padded_k(k), "invalid Q4/Q5/Q6 geometry");
    require(static_cast<std::int64_t>(tokens) * n < INT32_MAX, "Q4/Q5/Q6 output count exceeds int32");
    require(dtype == kF16, "the W4/5/6A16 matrix-core route takes FP16 activations");
    require(k % 8 == 0 && aligned(x, 16), "the W4/5/6A16 matrix-core route needs k % 8 == 0 and 16-byte aligned x");
    require(aligned(codes, 16) && aligned(scales, 4) && aligned(out, 2) && (bits == 4 || aligned(high, 16)),
            "misaligned Q4/Q5/Q6 operand");
    const auto* xp = static_cast<const __half*>(x);
    const auto* cp = static_cast<const std::uint8_t*>(codes);
    const auto* hp = static_cast<const std::uint8_t*>(high);
    const auto* sp = static_cast<const __half*>(scales);
    auto* op = static_cast<__half*>(out);
    if (tokens >= kRowPrefillMinTokens) {
        if (bits == 4) row_prefill_dispatch<0>(xp, cp, hp, sp, op, tokens, n, k, padded, stream);
        else if (bits == 5) row_prefill_dispatch<1>(xp, cp, hp, sp, op, tokens, n, k, padded, stream);
        else row_prefill_dispatch<2>(xp, cp, hp, sp, op, tokens, n, k, padded, stream);
        return;
    }
    if (bits == 4) row_decode_dispatch<0>(xp, cp, hp, sp, op, tokens, n, k, padded, stream);
    else if (bits == 5) row_decode_dispatch<1>(xp, cp, hp, sp, op, tokens, n, k, padded, stream);
    else row_decode_dispatch<2>(xp, cp, hp, sp, op, tokens, n, k, padded, stream);
}

// GW/GRB and DW/DRB: waves per workgroup and row blocks per wave of the
// gate/up and down GEMMs.
template <int GW, int GRB, int DW, int DRB, int NBMAX>
void moe_q4_launch_cfg(const void* x, const std::int64_t* ids, const void* scores, const void* gu_codes,
                       const void* gu_scales, const void* dn_codes, const void* dn_scales, void* out, void* workspace,
                       std::uint64_t workspace_bytes, int tokens, int top_k, int experts, int hidden, int inter,
                       hipStream_t stream) {
    moe_validate(tokens, top_k, experts, hidden, inter);
    require(x && ids && scores && gu_codes && gu_scales && dn_codes && dn_scales && out && workspace,
            "null MoE operand");
    const MoELayout l = moe_layout(tokens, top_k, experts, hidden, inter);
    require(workspace_bytes >= l.total, "MoE workspace is too small");
    require(aligned(x, 16) && aligned(out, 16) && aligned(workspace, 256) && aligned(ids, 8) && aligned(scores, 2),
            "misaligned MoE operand");
    require(aligned(gu_codes, 16) && aligned(dn_codes, 16) && aligned(gu_scales, 2) && aligned(dn_scales, 2),
            "misaligned Q4 expert plane");
    auto* ws = static_cast<std::uint8_t*>(workspace);
    int* seg = reinterpret_cast<int*>(ws + l.seg);
    int* status = reinterpret_cast<int*>(ws + l.status);
    int* pair_slot = reinterpret_cast<int*>(ws + l.pair_slot);
    int* slot_token = reinterpret_cast<int*>(ws + l.slot_token);
    auto* slot_score = reinterpret_cast<__half*>(ws + l.slot_score);
    auto* h = reinterpret_cast<__half*>(ws + l.h);
    auto* v = reinterpret_cast<__half*>(ws + l.v);
    const int pairs = tokens * top_k;

    // Up to kRouteList pairs the gate/up launch routes its experts itself (one
    // launch fewer); larger calls rank all pairs in moe_route first.
    const bool route_inside = pairs <= kRouteList;
    if (!route_inside)
        moe_route<<<1, kRouteThreads, 0, stream>>>(ids, static_cast<const __half*>(scores), pairs, top_k, experts,
                                                   seg, status, pair_slot, slot_token, slot_score);

    // Tiled planes: gate/up has ceil(inter/64) row tiles, down ceil(hidden/128);
    // chunks of 256 columns over the padded K.
    const int gu_chunks = static_cast<int>((padded_k(hidden) + kChunk - 1) / kChunk);
    const int dn_chunks = static_cast<int>((padded_k(inter) + kChunk - 1) / kChunk);
    Q4Tiled gu{};
    gu.x = static_cast<const __half*>(x);
    gu.gather = slot_token;
    gu.codes = static_cast<const uint4*>(gu_codes);
    gu.scales = static_cast<const __half*>(gu_scales);
    gu.row_tiles = (inter + kRows / 2 - 1) / (kRows / 2);
    gu.code_stride = static_cast<std::int64_t>(gu.row_tiles) * gu_chunks * kTileCodes;
    gu.scale_stride = static_cast<std::int64_t>(gu.row_tiles) * gu_chunks * 512;
    gu.seg = seg;
    gu.out = h;
    gu.n = 2 * inter;
    gu.k = hidden;
    gu.chunks = gu_chunks;
    gu.x_stride = hidden;
    gu.out_stride = inter;
    gu.experts = experts;
    gu.half_rows = inter;
    gu.ids = ids;
    gu.scores = static_cast<const __half*>(scores);
    gu.seg_out = seg;
    gu.status = status;
    gu.pair_slot = pair_slot;
    gu.slot_token = slot_token;
    gu.slot_score = slot_score;
    gu.pairs = pairs;
    gu.top_k = top_k;
    if (route_inside) launch_q4_grouped<kSwiGLU, GW, GRB, NBMAX, true, 1>(gu, stream);
    else launch_q4_grouped<kSwiGLU, GW, GRB, NBMAX, false, 1>(gu, stream);

    Q4Tiled dn{};
    dn.x = h;
    dn.codes = static_cast<const uint4*>(dn_codes);
    dn.scales = static_cast<const __half*>(dn_scales);
    dn.row_tiles = (hidden + kRows - 1) / kRows;
    dn.code_stride = static_cast<std::int64_t>(dn.row_tiles) * dn_chunks * kTileCodes;
    dn.scale_stride = static_cast<std::int64_t>(dn.row_tiles) * dn_chunks * 512;
    dn.seg = seg;
    dn.score = slot_score;
    dn.out = v;
    dn.n = hidden;
    dn.k = inter;
    dn.chunks = dn_chunks;
    dn.x_stride = inter;
    dn.out_stride = hidden;
    dn.experts = experts;
    launch_q4_grouped<kScore, DW, DRB, NBMAX, false, 2>(dn, stream);

    combine_dispatch(top_k, ids, pair_slot, v, static_cast<__half*>(out), tokens, hidden, stream);
}

void moe_q4_launch(const void* x, const std::int64_t* ids, const void* scores, const void* gu_codes,
                   const void* gu_scales, const void* dn_codes, const void* dn_scales, void* out, void* workspace,
                   std::uint64_t workspace_bytes, int tokens, int top_k, int experts, int hidden, int inter,
                   hipStream_t stream) {
    moe_q4_launch_cfg<8, 2, 8, 2, 3>(x, ids, scores, gu_codes, gu_scales, dn_codes, dn_scales, out, workspace,
                                     workspace_bytes, tokens, top_k, experts, hidden, inter, stream);
}

}  // namespace vt

#define VT_EXPORT extern "C" __attribute__((visibility("default")))

// Extension: the W4A16 contract GEMM on matrix cores (fp16 activations).
VT_EXPORT int venturi_q4_gemm_run(const void* x, const void* codes, const void* scales, void* out, int tokens, int n,
                                  int k, int padded, int dtype, void* stream) {
    return vt::guarded([&] {
        vt::row_gemm_launch(x, codes, nullptr, scales, out, tokens, n, k, padded, 4, dtype,
                            static_cast<hipStream_t>(stream));
    });
}

// Extension: exchange-slot bytes of venturi_q4_tiled_run (0 when the shape
// does not split K).
VT_EXPORT std::uint64_t venturi_q4_tiled_workspace_bytes(int tokens, int n, int k) {
    if (tokens <= 0 || n <= 0 || k <= 0) return 0;
    return vt::row_decode_slot_bytes(tokens, n, static_cast<int>(vt::padded_k(k)));
}

// Extension: puts a slot buffer in its idle state (once, before the first run;
// every run leaves its slots idle again).
VT_EXPORT int venturi_q4_tiled_workspace_init(void* workspace, std::uint64_t bytes, void* stream) {
    return vt::guarded([&] {
        vt::require(workspace && vt::aligned(workspace, 8) && bytes % 8 == 0, "invalid Q4 slot buffer");
        vt::fill_row_slot_buffer(static_cast<unsigned long long*>(workspace), bytes, static_cast<hipStream_t>(stream));
    });
}

// Extension: the W4A16 contract GEMM at decode token counts (1..31) over the
// tiled decode copy of q4.tile_q4 (contiguous wave loads; without a K split
// the same arithmetic and bits as venturi_q4_gemm_run on the row-major planes).
VT_EXPORT int venturi_q4_tiled_run(const void* x, const void* codes, const void* scales, void* out, int tokens, int n,
                                   int k, int padded, int dtype, void* workspace, std::uint64_t workspace_bytes,
                                   void* stream) {
    return vt::guarded([&] {
        vt::require(x && codes && scales && out, "null Q4 tiled operand");
        vt::require(tokens > 0 && tokens < vt::kRowPrefillMinTokens, "the tiled Q4 decode takes 1 to 31 tokens");
        vt::require(n > 0 && k > 0 && padded == vt::padded_k(k), "invalid Q4 geometry");
        vt::require(dtype == vt::kF16, "the tiled Q4 decode takes FP16 activations");
        vt::require(k % 8 == 0 && vt::aligned(x, 16), "the tiled Q4 decode needs k % 8 == 0 and 16-byte aligned x");
        vt::require(vt::aligned(codes, 16) && vt::aligned(scales, 4) && vt::aligned(out, 2),
                    "misaligned Q4 tiled operand");
        const std::uint64_t need = vt::row_decode_slot_bytes(tokens, n, padded);
        vt::require(workspace_bytes >= need && (need == 0 || (workspace && vt::aligned(workspace, 8))),
                    "the Q4 tiled decode needs its slot buffer (venturi_q4_tiled_workspace_bytes)");
        auto* slots = need ? static_cast<unsigned long long*>(workspace) : nullptr;
        vt::row_decode_dispatch<0, true>(static_cast<const __half*>(x), static_cast<const std::uint8_t*>(codes), nullptr,
                                         static_cast<const __half*>(scales), static_cast<__half*>(out), tokens, n, k,
                                         padded, static_cast<hipStream_t>(stream), slots);
        vt::settle_row_slots(slots, need, static_cast<hipStream_t>(stream));
    });
}

// Extension: venturi_q4_tiled_run for 4-, 5- and 6-bit row codecs (bits 4 reads
// the biased Q4 copy of q4.tile_q4, bits 5/6 the copy of q5.tile_row_codec with
// its tiled high plane); the slot buffer is sized by
// venturi_q4_tiled_workspace_bytes.
VT_EXPORT int venturi_row_tiled_run(const void* x, const void* codes, const void* high, const void* scales, void* out,
                                    int tokens, int n, int k, int padded, int bits, int dtype, void* workspace,
                                    std::uint64_t workspace_bytes, void* stream) {
    return vt::guarded([&] {
        vt::require(bits == 4 || bits == 5 || bits == 6, "row codecs are 4, 5 or 6 bits");
        vt::require(x && codes && scales && out && (bits == 4 || high), "null row-codec tiled operand");
        vt::require(tokens > 0 && tokens < vt::kRowPrefillMinTokens, "the tiled decode takes 1 to 31 tokens");
        vt::require(n > 0 && k > 0 && padded == vt::padded_k(k), "invalid row-codec geometry");
        vt::require(dtype == vt::kF16, "the tiled decode takes FP16 activations");
        vt::require(k % 8 == 0 && vt::aligned(x, 16), "the tiled decode needs k % 8 == 0 and 16-byte aligned x");
        vt::require(vt::aligned(codes, 16) && vt::aligned(scales, 4) && vt::aligned(out, 2) &&
                        (bits == 4 || vt::aligned(high, 4)),
                    "misaligned row-codec tiled operand");
        const std::uint64_t need = vt::row_decode_slot_bytes(tokens, n, padded);
        vt::require(workspace_bytes >= need && (need == 0 || (workspace && vt::aligned(workspace, 8))),
                    "the tiled decode needs its slot buffer (venturi_q4_tiled_workspace_bytes)");
        auto* slots = need ? static_cast<unsigned long long*>(workspace) : nullptr;
        const auto* xp = static_cast<const __half*>(x);
        const auto* cp = static_cast<const std::uint8_t*>(codes);
        const auto* hp = static_cast<const std::uint8_t*>(high);
        const auto* sp = static_cast<const __half*>(scales);
        auto* op = static_cast<__half*>(out);
        const hipStream_t st = static_cast<hipStream_t>(stream);
        if (bits == 4) vt::row_decode_dispatch<0, true>(xp, cp, nullptr, sp, op, tokens, n, k, padded, st, slots);
        else if (bits == 5) vt::row_decode_dispatch<1, true>(xp, cp, hp, sp, op, tokens, n, k, padded, st, slots);
        else vt::row_decode_dispatch<2, true>(xp, cp, hp, sp, op, tokens, n, k, padded, st, slots);
        vt::settle_row_slots(slots, need, st);
    });
}

// Extension: the W4A16 / W5A16 / W6A16 contract GEMM (fp16(q*scale) weights,
// fp32 accumulation on fp16 matrix cores) for 4-, 5- and 6-bit row codecs
// (q5/q6 read their high plane; `high` is unused for 4 bits).
VT_EXPORT int venturi_row_gemm_run(const void* x, const void* codes, const void* high, const void* scales, void* out,
                                   int tokens, int n, int k, int padded, int bits, int dtype, void* stream) {
    return vt::guarded([&] {
        vt::row_gemm_launch(x, codes, high, scales, out, tokens, n, k, padded, bits, dtype,
                            static_cast<hipStream_t>(stream));
    });
}

// Extension: workspace bytes of venturi_moe_q4_run (0 on invalid geometry).
VT_EXPORT std::uint64_t venturi_moe_q4_bytes(int tokens, int top_k, int experts, int hidden, int inter) {
    try {
        vt::moe_validate(tokens, top_k, experts, hidden, inter);
        return vt::moe_layout(tokens, top_k, experts, hidden, inter).total;
    } catch (const std::exception& e) {
        vt::set_error(e.what());
        return 0;
    }
}

// Extension: the routed-expert Q4 W4A16 MoE (flash_next_moe.py:139-161) in four
// launches: routing, gate/up GEMM with SiLU*up, down GEMM with the score,
// per-token combine. ids int64 [tokens][top_k], scores fp16 [tokens][top_k],
// expert planes stacked [experts][rows][...].
VT_EXPORT int venturi_moe_q4_run(const void* x, const std::int64_t* ids, const void* scores, const void* gu_codes,
                                 const void* gu_scales, const void* dn_codes, const void* dn_scales, void* out,
                                 void* workspace, std::uint64_t workspace_bytes, int tokens, int top_k, int experts,
                                 int hidden, int inter, void* stream) {
    return vt::guarded([&] {
        vt::moe_q4_launch(x, ids, scores, gu_codes, gu_scales, dn_codes, dn_scales, out, workspace, workspace_bytes,
                          tokens, top_k, experts, hidden, inter, static_cast<hipStream_t>(stream));
    });
}
