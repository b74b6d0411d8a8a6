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
// Schedule: the work items are the (position, group) pairs in visiting order
// (a position whose slot has no group is one item that only folds a zero
// sum). A step takes kBatch consecutive items, possibly spanning slots, so
// every step but the last is full whatever the number of groups per slot.
//
// Tiling: a 512-thread workgroup computes 128 tokens x 64 rows; wave
// (wm, wn) in 4 x 2 computes 32 x 32 as 2 x 2 MFMA tiles of 16 x 16. Each
// step's codes (converted to fp16) and scales are staged in one of two LDS
// buffers: a step computes from one buffer while the next step's operands,
// loaded during the previous step, are written to the other, with one barrier
// per step. LDS rows are group-major with an 80-byte stride, so the 16-byte
// fragment reads of 16 consecutive rows touch distinct banks. Within a step
// the fragments of the next item are read while an item's four products and
// its epilogue run; an item without data (past the end, or an empty slot) has
// its weight scale zeroed in LDS, so the epilogue runs unconditionally.
#include "common.hpp"

#include <algorithm>
#include <utility>

namespace vt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kTokTile = 128;
constexpr int kRowTile = 64;
constexpr int kRowHalves = 40;  // LDS row: 32 fp16 + 8 pad (80 bytes)

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

// Calls f(integral_constant<int, I>) for I = 0 .. N-1 (indices fixed at compile time).
template <class F, int... I>
__device__ __forceinline__ void for_each_index_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void for_each_index(F&& f) {
    for_each_index_impl(f, std::make_integer_sequence<int, N>{});
}

// Items per step: four with one pass; two with two passes (LDS budget).
template <int P>
struct A8Tile {
    static constexpr int kBatch = P == 1 ? 4 : 2;
};

template <int P>
__global__ __launch_bounds__(512) void a8_gemm(const std::int8_t* __restrict__ acodes,
                                               const float* __restrict__ ascales,
                                               const std::int8_t* __restrict__ wcodes,
                                               const __half* __restrict__ wscales, __half* __restrict__ out,
                                               int tokens, int n, int padded, int groups, int ldo) {
    constexpr int B = A8Tile<P>::kBatch;
    static_assert(B * kTokTile <= 512 && B * kRowTile <= 512, "one scale per thread and item");
    __shared__ __attribute__((aligned(16))) _Float16 af[2][P][B][kTokTile * kRowHalves];
    __shared__ __attribute__((aligned(16))) _Float16 bf[2][B][kRowTile * kRowHalves];
    __shared__ __attribute__((aligned(16))) float as_lds[2][P][B][kTokTile];
    __shared__ float ws_lds[2][B][kRowTile];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int q = lane >> 4, r = lane & 15;
    const int t0 = blockIdx.y * kTokTile, n0 = blockIdx.x * kRowTile;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;

    // Staging assignment (clamped rows are computed and never stored):
    // activation codes: token tid / 4, bytes 8 * (tid % 4) of every item's group;
    // weight codes: row tid / 8, bytes 4 * (tid % 8); activation scale: token
    // tid % 128 of item tid / 128; weight scale: row tid % 64 of item tid / 64.
    const std::int64_t a_tok = min(t0 + (tid >> 2), tokens - 1);
    const std::int8_t* a_src[P];
#pragma unroll
    for (int p = 0; p < P; ++p) a_src[p] = acodes + ((p * count) + a_tok * groups) * 32 + 8 * (tid & 3);
    const std::int8_t* b_src = wcodes + static_cast<std::int64_t>(min(n0 + (tid >> 3), n - 1)) * padded + 4 * (tid & 7);
    const int s_item = min(tid >> 7, B - 1);
    const int w_item = min(tid >> 6, B - 1);
    const float* as_src[P];
#pragma unroll
    for (int p = 0; p < P; ++p)
        as_src[p] = ascales + p * count + static_cast<std::int64_t>(min(t0 + (tid & 127), tokens - 1)) * groups;
    const __half* ws_src = wscales + static_cast<std::int64_t>(min(n0 + (tid & 63), n - 1)) * (padded / 32);

    // Schedule cursor: position p and item b within it. An item carries data
    // when its slot has groups (group bitrev5(p) + 32 b); the slot ends with
    // its last item (a position without groups has one item).
    struct Cursor {
        int p, b;
    };
    auto slot_groups = [&](int p) __attribute__((always_inline)) {
        const int slot = bitrev5(p);
        return slot < groups ? (groups - slot + 31) / 32 : 0;
    };

    struct Stage {
        uint2 a[P][B];
        std::uint32_t b[B];
        float as[P];
        unsigned short ws;
    };
    // Loads the operands of the B items at cursor c, advances it and returns
    // the step's descriptor: per item j, bits 8j (data), 8j+1 (slot ends) and
    // 8j+2..8j+6 (position). Items past the end load group groups - 1 and
    // have an empty descriptor.
    auto load = [&](Cursor& c, Stage& sg) __attribute__((always_inline)) {
        int gs = groups - 1, gw = groups - 1;
        std::uint32_t desc = 0;
        for_each_index<B>([&](auto J) __attribute__((always_inline)) {
            constexpr int j = decltype(J)::value;
            int g = groups - 1;
            if (c.p < 32) {
                const int cnt = slot_groups(c.p);
                std::uint32_t d = static_cast<std::uint32_t>(c.p) << 2;
                if (cnt > 0) {
                    g = bitrev5(c.p) + 32 * c.b;
                    d |= 1u;
                }
                if (c.b + 1 >= max(cnt, 1)) {
                    d |= 2u;
                    ++c.p;
                    c.b = 0;
                } else {
                    ++c.b;
                }
                desc |= d << (8 * j);
            }
#pragma unroll
            for (int p = 0; p < P; ++p) sg.a[p][j] = *reinterpret_cast<const uint2*>(a_src[p] + g * 32);
            sg.b[j] = *reinterpret_cast<const std::uint32_t*>(b_src + g * 32);
            gs = s_item == j ? g : gs;
            gw = w_item == j ? g : gw;
        });
#pragma unroll
        for (int p = 0; p < P; ++p) sg.as[p] = as_src[p][gs];
        sg.ws = __half_as_ushort(ws_src[gw]);
        return desc;
    };
    auto store = [&](const Stage& sg, std::uint32_t desc, int buf) __attribute__((always_inline)) {
        const int tok = tid >> 2;
#pragma unroll
        for (int j = 0; j < B; ++j) {
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const uint2 lo = codes4_to_half(sg.a[p][j].x), hi = codes4_to_half(sg.a[p][j].y);
                *reinterpret_cast<uint4*>(&af[buf][p][j][tok * kRowHalves + 8 * (tid & 3)]) =
                    make_uint4(lo.x, lo.y, hi.x, hi.y);
            }
            *reinterpret_cast<uint2*>(&bf[buf][j][(tid >> 3) * kRowHalves + 4 * (tid & 7)]) = codes4_to_half(sg.b[j]);
        }
        if (tid < B * kTokTile) {
#pragma unroll
            for (int p = 0; p < P; ++p) as_lds[buf][p][s_item][tid & 127] = sg.as[p];
        }
        // An item without data gets weight scale 0: its epilogue then adds
        // d * 0 to the slot sum, which leaves it unchanged (d is finite).
        if (tid < B * kRowTile)
            ws_lds[buf][w_item][tid & 63] = (desc >> (8 * w_item)) & 1u ? __half2float(__ushort_as_half(sg.ws)) : 0.0f;
    };

    float s[16], lv[5][16];
#pragma unroll
    for (int o = 0; o < 16; ++o) s[o] = 0.0f;
    // Fold the finished slot at position p into the level accumulators: a
    // level takes the first member of its pair and adds the second.
    auto fold = [&](int p) __attribute__((always_inline)) {
        if (p & 1) {
#pragma unroll
            for (int o = 0; o < 16; ++o) lv[0][o] += s[o];
            if (p & 2) {
#pragma unroll
                for (int o = 0; o < 16; ++o) lv[1][o] += lv[0][o];
                if (p & 4) {
#pragma unroll
                    for (int o = 0; o < 16; ++o) lv[2][o] += lv[1][o];
                    if (p & 8) {
#pragma unroll
                        for (int o = 0; o < 16; ++o) lv[3][o] += lv[2][o];
                        if (p & 16) {
#pragma unroll
                            for (int o = 0; o < 16; ++o) lv[4][o] += lv[3][o];
                        } else {
#pragma unroll
                            for (int o = 0; o < 16; ++o) lv[4][o] = lv[3][o];
                        }
                    } else {
#pragma unroll
                        for (int o = 0; o < 16; ++o) lv[3][o] = lv[2][o];
                    }
                } else {
#pragma unroll
                    for (int o = 0; o < 16; ++o) lv[2][o] = lv[1][o];
                }
            } else {
#pragma unroll
                for (int o = 0; o < 16; ++o) lv[1][o] = lv[0][o];
            }
        } else {
#pragma unroll
            for (int o = 0; o < 16; ++o) lv[0][o] = s[o];
        }
#pragma unroll
        for (int o = 0; o < 16; ++o) s[o] = 0.0f;
    };

    // Fragments of one item: activation codes and scales per pass and token
    // block, weight codes and scales per row block.
    struct Frag {
        half8 a[P][2];
        half8 b[2];
        float4 as[P][2];
        float ws[2];
    };
    auto read_frag = [&](int buf, int j, Frag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            f.ws[b] = ws_lds[buf][j][wn * 32 + 16 * b + r];
            f.b[b] = *reinterpret_cast<const half8*>(&bf[buf][j][(wn * 32 + 16 * b + r) * kRowHalves + 8 * q]);
        }
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                f.a[p][a] = *reinterpret_cast<const half8*>(&af[buf][p][j][(wm * 32 + 16 * a + r) * kRowHalves + 8 * q]);
                f.as[p][a] = *reinterpret_cast<const float4*>(&as_lds[buf][p][j][wm * 32 + 16 * a + 4 * q]);
            }
    };
    // Computes the B items of a step from LDS buffer buf. The fragments of
    // item j + 1 are read while item j's products and epilogue run.
    auto compute = [&](std::uint32_t desc, int buf) __attribute__((always_inline)) {
        const float4v zero = {0.0f, 0.0f, 0.0f, 0.0f};
        Frag f[2];
        read_frag(buf, 0, f[0]);
        for_each_index<B>([&](auto J) __attribute__((always_inline)) {
            constexpr int j = decltype(J)::value;
            const Frag& cur = f[j & 1];
            if constexpr (j + 1 < B) read_frag(buf, j + 1, f[(j + 1) & 1]);
            float4v d[P][2][2];
#pragma unroll
            for (int p = 0; p < P; ++p)
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int b = 0; b < 2; ++b)
                        d[p][a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.a[p][a], cur.b[b], zero, 0, 0, 0);
#pragma unroll
            for (int p = 0; p < P; ++p)
#pragma unroll
                for (int a = 0; a < 2; ++a) {
                    const float asv[4] = {cur.as[p][a].x, cur.as[p][a].y, cur.as[p][a].z, cur.as[p][a].w};
#pragma unroll
                    for (int b = 0; b < 2; ++b)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            float& acc = s[(a * 2 + b) * 4 + e];
                            acc = __fmaf_rn(d[p][a][b][e], __fmul_rn(cur.ws[b], asv[e]), acc);
                        }
                }
            const std::uint32_t item = desc >> (8 * j);
            if (item & 2u) fold(static_cast<int>((item >> 2) & 31u));
        });
    };

    // Items: one per (position, group), one per position without groups.
    // Operands of step t are loaded during step t - 2, written to LDS during
    // step t - 1 and consumed in step t.
    const int steps = (max(groups, 32) + B - 1) / B;
    static_assert(B <= 4, "four 8-bit item descriptors per word");
    Cursor cursor = {0, 0};
    Stage sg;
    std::uint32_t desc_now = load(cursor, sg), desc_next = 0;
    store(sg, desc_now, 0);
    if (steps > 1) desc_next = load(cursor, sg);
    __syncthreads();
    for (int step = 0; step < steps; ++step) {
        const int buf = step & 1;
        compute(desc_now, buf);
        desc_now = desc_next;
        if (step + 1 < steps) {
            store(sg, desc_now, buf ^ 1);  // operands of step + 1
            if (step + 2 < steps) desc_next = load(cursor, sg);
        }
        __syncthreads();
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
                    out[static_cast<std::int64_t>(t) * ldo + row] = from_f32<__half>(lv[4][(a * 2 + b) * 4 + e]);
            }
        }
}

}  // namespace

void a8_gemm_launch(const void* workspace, const std::int8_t* codes, const __half* scales, void* out, int tokens,
                    int n, int k, int padded, int passes, int ldo, hipStream_t stream) {
    const int groups = (k + 31) / 32;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const auto* acodes = static_cast<const std::int8_t*>(workspace);
    const auto* ascales = reinterpret_cast<const float*>(acodes + count * 32 * passes);
    const dim3 grid((n + kRowTile - 1) / kRowTile, (tokens + kTokTile - 1) / kTokTile);
    require(grid.y <= 65535, "token tiles exceed the launch grid");
    if (passes == 1)
        a8_gemm<1><<<grid, 512, 0, stream>>>(acodes, ascales, codes, scales, static_cast<__half*>(out), tokens, n,
                                              padded, groups, ldo);
    else
        a8_gemm<2><<<grid, 512, 0, stream>>>(acodes, ascales, codes, scales, static_cast<__half*>(out), tokens, n,
                                              padded, groups, ldo);
}

}  // namespace vt
