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
// chain stays in one lane in increasing column order. A wave processes RR
// rows and TT tokens at once so the activation words are reused RR times and
// the weight words TT times. The code*scale product is exact in fp32 (8-bit
// by 11-bit significands), so its evaluation order is immaterial.
#include "common.hpp"

namespace vt {
namespace {

constexpr int kWaves = 4;  // waves per 256-thread workgroup

template <class T>
__device__ __forceinline__ void load_x4(const T* x, std::int64_t base, int col, int k,
                                        bool vec, float (&xv)[4]);

template <>
__device__ __forceinline__ void load_x4<__half>(const __half* x, std::int64_t base, int col,
                                                int k, bool vec, float (&xv)[4]) {
    if (vec && col + 3 < k) {
        const uint2 w = *reinterpret_cast<const uint2*>(x + base + col);
        xv[0] = half_lo(w.x); xv[1] = half_hi(w.x);
        xv[2] = half_lo(w.y); xv[3] = half_hi(w.y);
    } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) xv[v] = col + v < k ? to_f32(x[base + col + v]) : 0.0f;
    }
}

template <>
__device__ __forceinline__ void load_x4<__hip_bfloat16>(const __hip_bfloat16* x, std::int64_t base,
                                                        int col, int k, bool vec, float (&xv)[4]) {
    if (vec && col + 3 < k) {
        const uint2 w = *reinterpret_cast<const uint2*>(x + base + col);
        xv[0] = bf16_lo(w.x); xv[1] = bf16_hi(w.x);
        xv[2] = bf16_lo(w.y); xv[3] = bf16_hi(w.y);
    } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) xv[v] = col + v < k ? to_f32(x[base + col + v]) : 0.0f;
    }
}

template <class T, int TT, int RR, bool VEC>
__global__ __launch_bounds__(256) void q8_exact(const T* __restrict__ x,
                                                const std::int8_t* __restrict__ codes,
                                                const __half* __restrict__ scales,
                                                T* __restrict__ out, int tokens, int n, int k,
                                                int padded) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * RR;
    const int t0 = blockIdx.y * TT;
    if (row0 >= n) return;
    const int groups = padded >> 5;

    float acc[TT][RR][4];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int r = 0; r < RR; ++r)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[t][r][v] = 0.0f;

    const std::uint32_t* wrow[RR];
    const __half* srow[RR];
#pragma unroll
    for (int r = 0; r < RR; ++r) {
        const int row = min(row0 + r, n - 1);  // clamped rows are computed, never stored
        wrow[r] = reinterpret_cast<const std::uint32_t*>(codes + static_cast<std::int64_t>(row) * padded);
        srow[r] = scales + static_cast<std::int64_t>(row) * groups;
    }

    for (int base = 0; base < k; base += 256) {
        const int col = base + 4 * lane;
        const bool live = col < k;
        std::uint32_t cw[RR];
        float s[RR];
#pragma unroll
        for (int r = 0; r < RR; ++r) {
            cw[r] = live ? wrow[r][col >> 2] : 0u;
            s[r] = live ? __half2float(srow[r][col >> 5]) : 0.0f;
        }
        float w[RR][4];
#pragma unroll
        for (int r = 0; r < RR; ++r)
#pragma unroll
            for (int v = 0; v < 4; ++v) w[r][v] = sbyte(cw[r], v) * s[r];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            if (t0 + t < tokens && live) {
                float xv[4];
                load_x4<T>(x, static_cast<std::int64_t>(t0 + t) * k, col, k, VEC, xv);
#pragma unroll
                for (int r = 0; r < RR; ++r)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        if (col + v < k) acc[t][r][v] = fmaf(xv[v], w[r][v], acc[t][r][v]);
            }
        }
    }

#pragma unroll
    for (int t = 0; t < TT; ++t) {
#pragma unroll
        for (int r = 0; r < RR; ++r) {
            const float y = canonical_sum(acc[t][r][0], acc[t][r][1], acc[t][r][2], acc[t][r][3]);
            if (lane == 0 && t0 + t < tokens && row0 + r < n)
                out[static_cast<std::int64_t>(t0 + t) * n + row0 + r] = from_f32<T>(y);
        }
    }
}

template <class T, int TT, int RR>
void launch_tile(const void* x, const std::int8_t* codes, const __half* scales, void* out,
                 int tokens, int n, int k, int padded, hipStream_t stream) {
    const dim3 grid((n + kWaves * RR - 1) / (kWaves * RR), (tokens + TT - 1) / TT);
    require(grid.y <= 65535, "token tiles exceed the launch grid");
    const bool vec = (k % 4 == 0) && aligned(x, 8);
    if (vec)
        q8_exact<T, TT, RR, true><<<grid, 256, 0, stream>>>(
            static_cast<const T*>(x), codes, scales, static_cast<T*>(out), tokens, n, k, padded);
    else
        q8_exact<T, TT, RR, false><<<grid, 256, 0, stream>>>(
            static_cast<const T*>(x), codes, scales, static_cast<T*>(out), tokens, n, k, padded);
}

template <class T>
void launch_exact(const void* x, const std::int8_t* codes, const __half* scales, void* out,
                  int tokens, int n, int k, int padded, hipStream_t stream) {
    if (tokens == 1) launch_tile<T, 1, 4>(x, codes, scales, out, tokens, n, k, padded, stream);
    else if (tokens == 2) launch_tile<T, 2, 4>(x, codes, scales, out, tokens, n, k, padded, stream);
    else if (tokens <= 4) launch_tile<T, 4, 2>(x, codes, scales, out, tokens, n, k, padded, stream);
    else if (tokens <= 8) launch_tile<T, 8, 2>(x, codes, scales, out, tokens, n, k, padded, stream);
    else launch_tile<T, 16, 1>(x, codes, scales, out, tokens, n, k, padded, stream);
}

__global__ void q8_embedding(const std::int8_t* codes, const __half* scales, const std::int64_t* ids,
                             void* out, int dtype, std::int64_t count, int vocab, int k, int padded) {
    // Reference: blocks.cu:293-304 (ids outside [0, vocab) read as zero rows).
    for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += static_cast<std::int64_t>(gridDim.x) * blockDim.x) {
        const std::int64_t row = ids[i / k];
        const int col = static_cast<int>(i % k);
        const float v = (row >= 0 && row < vocab)
                            ? static_cast<float>(codes[row * padded + col]) *
                                  __half2float(scales[row * (padded / 32) + col / 32])
                            : 0.0f;
        if (dtype == kF16) static_cast<__half*>(out)[i] = from_f32<__half>(v);
        else static_cast<__hip_bfloat16*>(out)[i] = from_f32<__hip_bfloat16>(v);
    }
}

void validate_q8(const void* x, const void* codes, const void* scales, const void* out, int tokens,
                 int n, int k, int padded) {
    require(x && codes && scales && out, "null Q8 operand");
    require(tokens > 0 && n > 0 && k > 0, "Q8 geometry must be positive");
    require(padded == padded_k(k), "padded K must equal ceil(k/128)*128");
    require(static_cast<std::int64_t>(tokens) * n < INT32_MAX, "Q8 output count exceeds int32");
    require(aligned(codes, 16), "Q8 codes require 16-byte alignment");
    require(aligned(scales, 2) && aligned(x, 2) && aligned(out, 2), "Q8 operands must be 2-byte aligned");
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
        const std::int64_t count = static_cast<std::int64_t>(tokens) * k;
        const int grid = static_cast<int>(std::min<std::int64_t>((count + 255) / 256, 65535));
        vt::q8_embedding<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(codes, scales, ids, out, dtype,
                                                                            count, vocab, k, padded);
    });
}

}  // extern "C"
