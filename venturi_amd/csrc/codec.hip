// Row-codec packing on the device.
//
// Q8 (q8_g32_fp16): the arithmetic of Q8RowSplitWeight.from_dense
// (ops/weights.py:398-439) for fp32-or-narrower sources: per 32-column group
// of the zero-padded row, scale = fp16(f32(max|x|) / 127) (IEEE division, then
// round-to-nearest-even); code = clamp(rint(x / f32(scale)), -127, 127), or 0
// when the stored scale is 0. The host rejects non-finite sources and scale
// overflow before launch, as the reference does.
//
// Q4 (q4_g64_fp16): the arithmetic of quantize_q4_rtn
// (models/flash_next/flash_next_q4.py:26-52): per 64-column group of the
// zero-padded row, scale = fp16(max(f32(max|x|) / 7, 2^-24)); code =
// clamp(rint(x / f32(scale)), -7, 7); groups wholly past k keep scale 0
// (from_codes zero-fills the plane past ceil(k/64)). Nibbles are packed two's
// complement, column 2j low (weights.py:108-130).
#include "common.hpp"

namespace vt {
namespace {

// Eight consecutive source values as fp32 from one 16-byte load (two for fp32).
__device__ __forceinline__ void load8(const __half* p, float (&v)[8]) {
    const uint4 w = *reinterpret_cast<const uint4*>(p);
    const std::uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = half_lo(u[i]);
        v[2 * i + 1] = half_hi(u[i]);
    }
}
__device__ __forceinline__ void load8(const __hip_bfloat16* p, float (&v)[8]) {
    const uint4 w = *reinterpret_cast<const uint4*>(p);
    const std::uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16_lo(u[i]);
        v[2 * i + 1] = bf16_hi(u[i]);
    }
}
__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}

// The 8 columns col .. col + 7 of a source row, zero past k. With `vec` (k % 8
// == 0 and a 16-byte aligned source) the 8 columns are all inside or all past
// k and come from one vector load; otherwise element by element.
template <class T>
__device__ __forceinline__ void row8(const T* __restrict__ row, int col, int k, bool vec, float (&v)[8]) {
    if (vec && col < k) {
        load8(row + col, v);
        return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = col + i < k ? to_f32(row[col + i]) : 0.0f;
}

// q[i] = rint(fl32(v[i] / d)) for 0 < d (the reference's fp32 division, then
// round half to even), without a division per value. r is the hardware
// reciprocal (1 ulp) refined by one Newton-Raphson step, r' = r + r (1 - d r),
// whose relative error is under 2^-24 + 2^-45 (the square of the reciprocal's
// plus one rounding); y = v * r' is then within |v/d| (2^-23 + 2^-44) of v/d,
// and fl32(v/d) within half an fp32 ulp of it. When every y lies farther than
// `guard` from the half-integers, each fl32(v/d) rounds as y does; otherwise
// the thread takes the IEEE division for all 8. Only quotients that the clamp
// does not decide matter (|v/d| < 8 for Q4, < 128 for Q8), where |y - fl32(v/d)|
// stays under 1.5 * 2^-20 and 1.25 * 2^-16: the guards of 2^-17 and 2^-14 leave
// margins above 5x and 3x. A NaN estimate (non-finite source) takes the division.
__device__ __forceinline__ void rint_quotients(const float (&v)[8], float d, float guard, float (&q)[8]) {
    const float r0 = __builtin_amdgcn_rcpf(d);
    const float r = fmaf(r0, fmaf(-d, r0, 1.0f), r0);
    bool near = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float y = v[i] * r;
        q[i] = rintf(y);
        near |= !(fabsf(y - q[i]) < 0.5f - guard);
    }
    if (near) {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = rintf(__fdiv_rn(v[i], d));
    }
}

template <class T>
__global__ __launch_bounds__(256) void q8_pack(const T* __restrict__ src, std::int8_t* __restrict__ codes,
                                               __half* __restrict__ scales, int n, int k, int padded, bool vec) {
    // 4 lanes per group, 8 consecutive columns per lane.
    const int groups = padded >> 5;
    const std::int64_t index = (static_cast<std::int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 2;
    const int sub = threadIdx.x & 3;
    if (index >= static_cast<std::int64_t>(n) * groups) return;  // a group's 4 lanes exit together
    const std::int64_t row = index / groups;
    const int col = static_cast<int>(index % groups) * 32 + sub * 8;
    float v[8];
    row8(src + row * k, col, k, vec, v);
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[i]));
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    const __half stored = from_f32<__half>(__fdiv_rn(mx, 127.0f));
    const float d = __half2float(stored);
    float qf[8];
    rint_quotients(v, d > 0.0f ? d : 1.0f, 0x1p-14f, qf);
    std::uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int q = d > 0.0f ? static_cast<int>(fminf(fmaxf(qf[i], -127.0f), 127.0f)) : 0;
        const std::uint32_t byte = static_cast<std::uint32_t>(q & 0xff) << (8 * (i & 3));
        if (i < 4) lo |= byte; else hi |= byte;
    }
    *reinterpret_cast<uint2*>(codes + row * padded + col) = make_uint2(lo, hi);
    if (sub == 0) scales[index] = stored;
}

template <class T>
__global__ __launch_bounds__(256) void q4_pack(const T* __restrict__ src, std::uint8_t* __restrict__ codes,
                                               __half* __restrict__ scales, int n, int k, int padded, bool vec) {
    // 8 lanes per 64-column group, 8 consecutive columns (4 code bytes) per lane.
    const int groups = padded >> 6;
    const std::int64_t index = (static_cast<std::int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 3;
    const int sub = threadIdx.x & 7;
    if (index >= static_cast<std::int64_t>(n) * groups) return;  // a group's 8 lanes exit together
    const std::int64_t row = index / groups;
    const int group = static_cast<int>(index % groups);
    const int col = group * 64 + sub * 8;
    float v[8];
    row8(src + row * k, col, k, vec, v);
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[i]));
    mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 4, 64));
    const bool live = group * 64 < k;
    const __half stored = live ? from_f32<__half>(fmaxf(__fdiv_rn(mx, 7.0f), 0x1p-24f)) : __float2half(0.0f);
    const float d = __half2float(stored);
    float qf[8];
    rint_quotients(v, live ? d : 1.0f, 0x1p-17f, qf);
    std::uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int q = live ? static_cast<int>(fminf(fmaxf(qf[i], -7.0f), 7.0f)) : 0;
        word |= static_cast<std::uint32_t>(q & 15) << (4 * i);
    }
    *reinterpret_cast<std::uint32_t*>(codes + row * (padded / 2) + col / 2) = word;
    if (sub == 0) scales[index] = stored;
}

}  // namespace
}  // namespace vt

// Extension (the reference quantizes Q4 on the CPU only): device
// quantize_q4_rtn of an [n, k] fp16/bf16/fp32 matrix into codes [n][padded/2]
// and scales [n][padded/64].
extern "C" __attribute__((visibility("default"))) int venturi_q4_pack_run(const void* src, void* codes, void* scales,
                                                                         int n, int k, int padded, int dtype,
                                                                         void* stream) {
    return vt::guarded([&] {
        vt::require(src && codes && scales && n > 0 && k > 0 && padded == vt::padded_k(k), "invalid Q4 pack geometry");
        vt::require(vt::aligned(codes, 4) && vt::aligned(scales, 2), "Q4 pack outputs must be aligned");
        const std::int64_t lanes = static_cast<std::int64_t>(n) * (padded / 64) * 8;
        const std::int64_t blocks = (lanes + 255) / 256;
        vt::require(blocks <= INT32_MAX, "Q4 pack grid too large");
        auto s = static_cast<hipStream_t>(stream);
        auto* c = static_cast<std::uint8_t*>(codes);
        auto* sc = static_cast<__half*>(scales);
        const unsigned grid = static_cast<unsigned>(blocks);
        const bool vec = k % 8 == 0 && vt::aligned(src, 16);
        if (dtype == vt::kF16)
            vt::q4_pack<<<grid, 256, 0, s>>>(static_cast<const __half*>(src), c, sc, n, k, padded, vec);
        else if (dtype == vt::kBF16)
            vt::q4_pack<<<grid, 256, 0, s>>>(static_cast<const __hip_bfloat16*>(src), c, sc, n, k, padded, vec);
        else if (dtype == vt::kF32)
            vt::q4_pack<<<grid, 256, 0, s>>>(static_cast<const float*>(src), c, sc, n, k, padded, vec);
        else
            throw vt::Invalid("unsupported source dtype");
    });
}

// Extension (the reference packs on the CPU only): device Q8 packing of an
// [n, k] fp16/bf16/fp32 matrix into codes [n][padded] and scales [n][padded/32].
extern "C" __attribute__((visibility("default"))) int venturi_q8_pack_run(const void* src, std::int8_t* codes,
                                                                         void* scales, int n, int k, int padded,
                                                                         int dtype, void* stream) {
    return vt::guarded([&] {
        vt::require(src && codes && scales && n > 0 && k > 0 && padded == vt::padded_k(k), "invalid Q8 pack geometry");
        vt::require(vt::aligned(codes, 8) && vt::aligned(scales, 2), "Q8 pack outputs must be aligned");
        const std::int64_t lanes = static_cast<std::int64_t>(n) * (padded / 32) * 4;
        const std::int64_t blocks = (lanes + 255) / 256;
        vt::require(blocks <= INT32_MAX, "Q8 pack grid too large");
        auto s = static_cast<hipStream_t>(stream);
        auto* sc = static_cast<__half*>(scales);
        const bool vec = k % 8 == 0 && vt::aligned(src, 16);
        const unsigned grid = static_cast<unsigned>(blocks);
        if (dtype == vt::kF16)
            vt::q8_pack<<<grid, 256, 0, s>>>(static_cast<const __half*>(src), codes, sc, n, k, padded, vec);
        else if (dtype == vt::kBF16)
            vt::q8_pack<<<grid, 256, 0, s>>>(static_cast<const __hip_bfloat16*>(src), codes, sc, n, k, padded, vec);
        else if (dtype == vt::kF32)
            vt::q8_pack<<<grid, 256, 0, s>>>(static_cast<const float*>(src), codes, sc, n, k, padded, vec);
        else
            throw vt::Invalid("unsupported source dtype");
    });
}
