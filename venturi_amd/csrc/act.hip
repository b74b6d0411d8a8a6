// Elementwise SwiGLU and add of the native runtime (blocks.cu:56-86, 741-750):
//   swiglu: out = cast((x * sigmoid(x)) * y) in fp32, one rounding at the end,
//           sigmoid(x) = x >= 0 ? 1 / (1 + exp(-x)) : exp(x) / (1 + exp(x));
//   add:    out = cast(x + y).
// `venturi_silu_mul_run` applies the same SwiGLU to one fused gate/up buffer
// [tokens][2*inter] (the output of a fused gate+up projection).
#include "common.hpp"

namespace vt {
namespace {

template <class T, bool SWIGLU>
__global__ __launch_bounds__(256) void elementwise(const T* __restrict__ a, const T* __restrict__ b, T* __restrict__ out,
                                                   std::int64_t count) {
    for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * 256 + threadIdx.x; i < count;
         i += static_cast<std::int64_t>(gridDim.x) * 256) {
        const float x = to_f32(a[i]), y = to_f32(b[i]);
        out[i] = from_f32<T>(SWIGLU ? swiglu_value(x, y) : __fadd_rn(x, y));
    }
}

template <class T>
__global__ __launch_bounds__(256) void swiglu_fused(const T* __restrict__ gate_up, T* __restrict__ out, int tokens,
                                                    int inter) {
    const std::int64_t total = static_cast<std::int64_t>(tokens) * inter;
    for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += static_cast<std::int64_t>(gridDim.x) * 256) {
        const std::int64_t t = i / inter;
        const int c = static_cast<int>(i % inter);
        out[i] = from_f32<T>(swiglu_value(to_f32(gate_up[t * 2 * inter + c]), to_f32(gate_up[t * 2 * inter + inter + c])));
    }
}

unsigned grid_for(std::int64_t count) { return static_cast<unsigned>(std::min<std::int64_t>((count + 255) / 256, 65535)); }

template <bool SWIGLU>
void launch_elementwise(const void* a, const void* b, void* out, std::int64_t count, int dtype, hipStream_t stream) {
    require(a && b && out && count > 0, "invalid element count");
    const unsigned grid = grid_for(count);
    if (dtype == kF16)
        elementwise<__half, SWIGLU><<<grid, 256, 0, stream>>>(static_cast<const __half*>(a), static_cast<const __half*>(b),
                                                              static_cast<__half*>(out), count);
    else if (dtype == kBF16)
        elementwise<__hip_bfloat16, SWIGLU><<<grid, 256, 0, stream>>>(static_cast<const __hip_bfloat16*>(a),
                                                                      static_cast<const __hip_bfloat16*>(b),
                                                                      static_cast<__hip_bfloat16*>(out), count);
    else if (dtype == kF32)
        elementwise<float, SWIGLU><<<grid, 256, 0, stream>>>(static_cast<const float*>(a), static_cast<const float*>(b),
                                                             static_cast<float*>(out), count);
    else
        throw Invalid("unsupported scalar type");
}

}  // namespace
}  // namespace vt

#define VT_EXPORT extern "C" __attribute__((visibility("default")))

// Reference: blocks.cu:741-745 (dtype 0/1/2; fp32 math, one rounding).
VT_EXPORT int venturi_swiglu_run(const void* a, const void* b, void* out, std::int64_t count, int dtype, void* stream) {
    return vt::guarded([&] { vt::launch_elementwise<true>(a, b, out, count, dtype, static_cast<hipStream_t>(stream)); });
}

// Reference: blocks.cu:746-750.
VT_EXPORT int venturi_add_run(const void* a, const void* b, void* out, std::int64_t count, int dtype, void* stream) {
    return vt::guarded([&] { vt::launch_elementwise<false>(a, b, out, count, dtype, static_cast<hipStream_t>(stream)); });
}

// Extension: the same SwiGLU over a fused gate+up output [tokens][2*inter]
// (gate columns first) into out [tokens][inter]; dtype 0 or 1.
VT_EXPORT int venturi_silu_mul_run(const void* gate_up, void* out, int tokens, int inter, int dtype, void* stream) {
    return vt::guarded([&] {
        vt::require(gate_up && out && tokens > 0 && inter > 0, "invalid SiLU*up operands");
        const std::int64_t total = static_cast<std::int64_t>(tokens) * inter;
        const unsigned grid = vt::grid_for(total);
        auto s = static_cast<hipStream_t>(stream);
        if (dtype == vt::kF16)
            vt::swiglu_fused<<<grid, 256, 0, s>>>(static_cast<const __half*>(gate_up), static_cast<__half*>(out), tokens,
                                                  inter);
        else if (dtype == vt::kBF16)
            vt::swiglu_fused<<<grid, 256, 0, s>>>(static_cast<const __hip_bfloat16*>(gate_up),
                                                  static_cast<__hip_bfloat16*>(out), tokens, inter);
        else
            throw vt::Invalid("SiLU*up takes fp16 or bf16");
    });
}
