// Shared host/device helpers for the gfx950 quantized-linear library.
//
// Every exported entry point follows one contract: validate geometry and
// pointers on the host, launch on the caller's stream, return 0 on success or
// -1 with a per-thread message readable through venturi_blocks_error().
// Nothing here allocates device memory or synchronises (the dense route's
// one-time hipBLASLt set-up per device and shape aside).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace vt {

// Per-thread error text (defined once in api.cpp).
void set_error(const char* text);
void clear_error();

struct Invalid : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};

inline void require(bool ok, const char* message) {
    if (!ok) throw Invalid(message);
}

inline void check(hipError_t status) {
    if (status != hipSuccess) throw std::runtime_error(hipGetErrorString(status));
}

inline bool aligned(const void* p, std::uintptr_t bytes) {
    return (reinterpret_cast<std::uintptr_t>(p) % bytes) == 0;
}

inline std::int64_t padded_k(std::int64_t k) { return (k + 127) / 128 * 128; }

// Runs `body`, mapping exceptions to the -1 / message convention.
template <class F>
int guarded(F&& body) {
    try {
        clear_error();
        body();
        check(hipGetLastError());
        return 0;
    } catch (const std::exception& e) {
        set_error(e.what());
        return -1;
    }
}

// Host-only variant for entry points that make no HIP call (sizes, admission):
// maps exceptions to the message convention without touching the runtime.
template <class F>
bool host_guarded(F&& body) {
    try {
        clear_error();
        body();
        return true;
    } catch (const std::exception& e) {
        set_error(e.what());
        return false;
    }
}

// Activation scalar types selected by the reference's dtype codes
// (0 = fp16, 1 = bf16, 2 = fp32).
enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

__device__ __forceinline__ float to_f32(__half v) { return __half2float(v); }
__device__ __forceinline__ float to_f32(__hip_bfloat16 v) { return __bfloat162float(v); }
__device__ __forceinline__ float to_f32(float v) { return v; }

// The reference rounds every result to fp32 first and then to the 16-bit
// output type (two roundings). Without a barrier LLVM folds fp16(a*b) or
// fp16(a+b) into v_fma_mixlo_f16, which rounds once, straight to fp16, and
// differs in rare double-rounding cases; the empty asm pins the fp32 value.
__device__ __forceinline__ float f32_pin(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

template <class T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ __half from_f32<__half>(float v) { return __float2half_rn(f32_pin(v)); }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float v) {
    return __float2bfloat16(f32_pin(v));  // round-to-nearest-even
}
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }

// Bit-level fp16 decode of the low/high half of a 32-bit word.
__device__ __forceinline__ float half_lo(std::uint32_t w) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(w & 0xffffu)));
}
__device__ __forceinline__ float half_hi(std::uint32_t w) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(w >> 16)));
}
__device__ __forceinline__ float bf16_lo(std::uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(std::uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Weight-stream loads. Decode kernels read every weight byte once per launch,
// so the loads carry the non-temporal hint (global_load ... nt): on MI355X a
// streaming read with it measured 5-9% faster at 33-189 MB than the default
// policy (189 MB: 30.3 -> 27.8 us; 94 MB: 16.0 -> 14.7 us), the lines not
// competing with activations and outputs for L2.
__device__ __forceinline__ uint4 stream_load(const uint4* p) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ std::uint32_t stream_load(const std::uint32_t* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ unsigned short stream_load(const unsigned short* p) {
    return __builtin_nontemporal_load(p);
}

// Sign-extending byte extraction from a packed int8x4 word.
__device__ __forceinline__ float sbyte(std::uint32_t w, int i) {
    return static_cast<float>(static_cast<std::int8_t>(w >> (8 * i)));
}

// Correctly rounded square root. hipcc lowers __builtin_sqrtf for gfx950 to
// v_sqrt_f32 followed by an exact neighbour correction (checked bit-for-bit
// against IEEE sqrt on 16.8M random normal inputs); __fsqrt_rn does not
// correct and is up to one ulp off, so it is not used.
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }

// SwiGLU of the native runtime (blocks.cu:56-86): (x * sigmoid(x)) * y in fp32
// with the reference's stable logistic; expf is the ROCm device library's (its
// last bit is not pinned against CUDA's; the final cast absorbs it almost
// always). Shared by the elementwise kernels and the fused projection epilogue.
__device__ __forceinline__ float swiglu_value(float x, float y) {
    const float sigmoid = x >= 0.0f ? __fdiv_rn(1.0f, 1.0f + expf(-x)) : __fdiv_rn(expf(x), 1.0f + expf(x));
    return __fmul_rn(__fmul_rn(x, sigmoid), y);
}

// v from lane (lane + N) of the same 16-lane row (DPP row_shl:N; lanes whose
// source lies past the row read 0).
template <int N>
__device__ __forceinline__ float row_shl(float v) {
    static_assert(N >= 1 && N <= 15, "DPP row shifts move 1..15 lanes");
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x100 + N, 0xF, 0xF, true));
}

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// The reference's 256-thread reduction (cuda_common.cuh:38-51, block_sum)
// applied to 256 "virtual threads" held four per lane: lane L holds the
// partials of threads 4L..4L+3 in a0..a3. Threads 32w..32w+31 (lanes
// 8w..8w+7) are first summed by the shfl_down 16/8/4/2/1 tree over
// t = 4*(lane%8) + v, i.e. lane offsets +4, +2, +1 and then register pairs
// (+2, +1). The eight group sums are then reduced by the same tree run over
// 32 lanes of which only 0..7 are nonzero: the +16 and +8 steps add exact
// zeros, the +4/+2/+1 steps pair group sums g + 4, then + 2, then + 1 (held
// in lanes 8g). The lane offsets +4/+2/+1 stay inside a 16-lane row, so they
// are DPP row shifts (the lanes that feed the group sums read only lanes of
// their own group); the eight group sums are read into scalars and paired in
// the tree's order. Every addition is the reference's, in its order, so the
// bits are the same. Returns the same value in every lane; all lanes of the
// wave must call it together.
__device__ __forceinline__ float canonical_sum(float a0, float a1, float a2, float a3) {
    a0 += row_shl<4>(a0); a1 += row_shl<4>(a1); a2 += row_shl<4>(a2); a3 += row_shl<4>(a3);
    a0 += row_shl<2>(a0); a1 += row_shl<2>(a1); a2 += row_shl<2>(a2); a3 += row_shl<2>(a3);
    a0 += row_shl<1>(a0); a1 += row_shl<1>(a1); a2 += row_shl<1>(a2); a3 += row_shl<1>(a3);
    float p = (a0 + a2) + (a1 + a3);
    p = (p + 0.0f) + 0.0f;
    const float g04 = lane_value(p, 0) + lane_value(p, 32), g26 = lane_value(p, 16) + lane_value(p, 48);
    const float g15 = lane_value(p, 8) + lane_value(p, 40), g37 = lane_value(p, 24) + lane_value(p, 56);
    return (g04 + g26) + (g15 + g37);
}

// 32-lane shfl_down 16/8/4/2/1 tree (one reference warp per half-wave);
// valid in lanes 0 and 32. The +16 step crosses a 16-lane row (one LDS
// permute); the +8/+4/+2/+1 steps that lanes 0 and 32 depend on read only
// lanes of their own row, so they are DPP row shifts. Same additions, same
// order. All lanes of the wave must call it together.
__device__ __forceinline__ float warp32_sum(float v) {
    v += __shfl_down(v, 16, 32);
    v += row_shl<8>(v);
    v += row_shl<4>(v);
    v += row_shl<2>(v);
    v += row_shl<1>(v);
    return v;
}

// GEMM tile shapes of the prefill kernels: each candidate is one workgroup of
// 8 waves per CU; pick_tiling returns the one with the least time over whole
// tile rounds on the device's CUs, from the candidates' measured rates per
// unit of work (a tile round costs tm * tn / rate).
struct GemmTiling {
    int tm, tn;
    double rate;
};

inline int device_cus() {
    static const int cus = [] {
        int device = 0, count = 0;
        check(hipGetDevice(&device));
        check(hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device));
        return count > 0 ? count : 1;
    }();
    return cus;
}

template <int N>
inline int pick_tiling(int tokens, int n, const GemmTiling (&tilings)[N]) {
    const int cus = device_cus();
    int best = 0;
    double best_cost = 0.0;
    for (int i = 0; i < N; ++i) {
        const GemmTiling& t = tilings[i];
        const std::int64_t tiles =
            static_cast<std::int64_t>((tokens + t.tm - 1) / t.tm) * ((n + t.tn - 1) / t.tn);
        const double cost = static_cast<double>((tiles + cus - 1) / cus) * t.tm * t.tn / t.rate;
        if (i == 0 || cost < best_cost) {
            best = i;
            best_cost = cost;
        }
    }
    return best;
}

}  // namespace vt
