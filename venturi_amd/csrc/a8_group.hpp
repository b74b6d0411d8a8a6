// Per-32-group int8 activation quantization (q8_dp4a.cuh:15-34), shared by
// the quantizer kernels and the A8 decode kernel that quantizes its own
// activations.
#pragma once

#include "common.hpp"

namespace vt {
namespace {

// Whether any of a group's values is non-finite: GL adjacent lanes hold the
// group (their flags are combined across the lanes).
template <int GL>
__device__ __forceinline__ bool group_invalid(bool bad_local) {
    int bad = bad_local ? 1 : 0;
#pragma unroll
    for (int m = 1; m < GL; m <<= 1) bad |= __shfl_xor(bad, m, 64);
    return bad != 0;
}

// One pass over a group whose 32 values sit NV per lane on GL adjacent lanes
// (NV*GL == 32): the group max is order independent; the scale and inverse
// are IEEE f32 divisions, the code is the RNE f32 product rounded
// half-to-even and clamped to +-127, and the residual update is one fused
// multiply-add, exactly as the reference. `word` receives the lane's NV codes
// (four per 32-bit word, lowest column first), `r` the residual; returns the
// scale as stored (NaN for an invalid group, whose codes are all zero).
template <int NV, int GL>
__device__ __forceinline__ float quantize_pass(float (&r)[NV], bool invalid, std::uint32_t (&word)[NV / 4]) {
    static_assert(NV * GL == 32, "a group is 32 values");
    float mx = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; ++v) mx = fmaxf(mx, fabsf(r[v]));
#pragma unroll
    for (int m = 1; m < GL; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    const float scale = __fdiv_rn(mx, 127.0f);
    const float inverse = mx > 0.0f ? __fdiv_rn(127.0f, mx) : 0.0f;
#pragma unroll
    for (int i = 0; i < NV / 4; ++i) word[i] = 0u;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        int code = 0;
        if (!invalid) {
            const float scaled = rintf(__fmul_rn(r[v], inverse));
            code = static_cast<int>(fminf(fmaxf(scaled, -127.0f), 127.0f));
        }
        word[v / 4] |= static_cast<std::uint32_t>(code & 0xff) << (8 * (v % 4));
        r[v] = __fmaf_rn(-static_cast<float>(code), scale, r[v]);
    }
    return invalid ? __builtin_nanf("") : scale;
}

// All passes of a group, stored in the workspace layout: codes at
// codes_out + p * code_pass_stride (NV bytes per lane), the scale at
// scale_out + p * scale_pass_stride by the group's leader lane. A group with
// any non-finite input stores zero codes and a NaN scale for every pass.
template <int NV, int GL>
__device__ __forceinline__ void quantize_group(float (&r)[NV], bool bad_local, int passes,
                                               std::int8_t* codes_out, float* scale_out,
                                               std::int64_t code_pass_stride,
                                               std::int64_t scale_pass_stride, bool leader) {
    const bool invalid = group_invalid<GL>(bad_local);
    for (int p = 0; p < passes; ++p) {
        std::uint32_t word[NV / 4];
        const float scale = quantize_pass<NV, GL>(r, invalid, word);
        std::int8_t* dst = codes_out + p * code_pass_stride;
        if constexpr (NV == 4) {
            *reinterpret_cast<std::uint32_t*>(dst) = word[0];
        } else {
            static_assert(NV == 8, "4 or 8 values per lane");
            *reinterpret_cast<uint2*>(dst) = make_uint2(word[0], word[1]);
        }
        if (leader) scale_out[p * scale_pass_stride] = scale;
    }
}

}  // namespace
}  // namespace vt
