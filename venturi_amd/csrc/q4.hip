// Q4 (q4_g64_fp16) row codec on gfx950: fp16 decode, the reference's two Q4
// decode projections in their exact orders, and a W4A16 matrix-core GEMM.
//
// Layout: codes uint8 [n][padded/2], column 2j in the low nibble of byte j,
// two's-complement q in [-8, 7]; scales fp16 [n][padded/64].
//
// Weight values (reference):
//  * expert / W4A16 contract: w = fp16(q * scale) rounded to nearest even
//    (flash_next_q4.cu:7-14, quantization/linear.py:86-95);
//  * plugin contract (q4_linear.cu:21-56): w = f32(q) * f32(scale), exact in
//    fp32 (4-bit by 11-bit significands).
#include "common.hpp"

#include <algorithm>

namespace vt {
namespace {

__device__ __forceinline__ int nibble(std::uint32_t word, int i) {
    const int u = static_cast<int>((word >> (4 * i)) & 15u);
    return (u ^ 8) - 8;
}

// ---------------------------------------------------------------------------
// fp16 decode: each thread writes 8 columns (one code word of 4 bytes).
__global__ __launch_bounds__(256) void q4_decode(const std::uint8_t* __restrict__ codes,
                                                 const __half* __restrict__ scales, __half* __restrict__ out,
                                                 int row_begin, int rows, int k, int padded) {
    const int local = blockIdx.y;
    const int col = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (local >= rows || col >= k) return;
    const std::int64_t row = static_cast<std::int64_t>(row_begin) + local;
    const std::uint8_t* c = codes + row * (padded / 2) + col / 2;
    const std::uint32_t word = *reinterpret_cast<const std::uint32_t*>(c);  // col % 8 == 0: 4-byte aligned
    const float s = __half2float(scales[row * (padded / 64) + col / 64]);
    unsigned short h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = __half_as_ushort(from_f32<__half>(static_cast<float>(nibble(word, j)) * s));
    __half* d = out + static_cast<std::int64_t>(local) * k + col;
    if (col + 7 < k && (reinterpret_cast<std::uintptr_t>(d) & 15) == 0) {
        *reinterpret_cast<uint4*>(d) =
            make_uint4(h[0] | (static_cast<std::uint32_t>(h[1]) << 16), h[2] | (static_cast<std::uint32_t>(h[3]) << 16),
                       h[4] | (static_cast<std::uint32_t>(h[5]) << 16), h[6] | (static_cast<std::uint32_t>(h[7]) << 16));
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (col + j < k) d[j] = __ushort_as_half(h[j]);
    }
}

// ---------------------------------------------------------------------------
// Expert GEMV (flash_next_q4.cu:23-34): for output (t, row) lane l of a
// 32-lane reference warp accumulates sum = fmaf(w(col), x[col], sum) over
// col = l, l+32, ... < cols with w = fp16(q*scale), then a shfl_down
// 16/8/4/2/1 tree; fp16 output. (The reference writes sum += w*x, which
// nvcc contracts to that fmaf.) One half-wave per (row, token).
__global__ __launch_bounds__(256) void q4_linear_exact(const __half* __restrict__ x,
                                                       const std::uint8_t* __restrict__ codes,
                                                       const __half* __restrict__ scales, __half* __restrict__ out,
                                                       int rows, int cols, int padded) {
    const int lane = threadIdx.x & 31;
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int token = blockIdx.y;
    float sum = 0.0f;
    if (row < rows) {
        const std::uint8_t* c = codes + static_cast<std::int64_t>(row) * (padded / 2);
        const __half* s = scales + static_cast<std::int64_t>(row) * (padded / 64);
        const __half* xr = x + static_cast<std::int64_t>(token) * cols;
        for (int col = lane; col < cols; col += 32) {
            const int q = nibble(c[col >> 1], col & 1);
            const float w = __half2float(from_f32<__half>(static_cast<float>(q) * __half2float(s[col >> 6])));
            sum = fmaf(w, __half2float(xr[col]), sum);
        }
    }
    sum = warp32_sum(sum);
    if (lane == 0 && row < rows) out[static_cast<std::int64_t>(token) * rows + row] = from_f32<__half>(sum);
}

// ---------------------------------------------------------------------------
// Plugin GEMV (q4_linear.cu:21-56): lane l of a 32-lane warp owns byte l of
// every 32-byte group, i.e. columns 64g+2l and 64g+2l+1, with fp32 weights
// q*scale; per token sum = fmaf(x0, w0, sum) then fmaf(x1, w1, sum) in
// increasing g, then the 32-lane tree; RNE cast to the activation type.
// One half-wave per row, four tokens per half-wave.
template <class T>
__global__ __launch_bounds__(256) void q4_generic_exact(const T* __restrict__ x, const std::uint8_t* __restrict__ codes,
                                                        const __half* __restrict__ scales, T* __restrict__ out, int n,
                                                        int k, int padded, int tokens) {
    const int lane = threadIdx.x & 31;
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int t0 = blockIdx.y * 4;
    float sums[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (row < n) {
        const std::uint8_t* c = codes + static_cast<std::int64_t>(row) * (padded / 2);
        const __half* s = scales + static_cast<std::int64_t>(row) * (padded / 64);
        const int groups = (k + 63) / 64;
        for (int g = 0; g < groups; ++g) {
            const std::uint32_t byte = c[g * 32 + lane];
            const float scale = __half2float(s[g]);
            const float w0 = static_cast<float>(nibble(byte, 0)) * scale;
            const float w1 = static_cast<float>(nibble(byte, 1)) * scale;
            const int col = g * 64 + 2 * lane;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (t0 + t < tokens) {
                    const T* xr = x + static_cast<std::int64_t>(t0 + t) * k;
                    if (col < k) sums[t] = fmaf(to_f32(xr[col]), w0, sums[t]);
                    if (col + 1 < k) sums[t] = fmaf(to_f32(xr[col + 1]), w1, sums[t]);
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float y = warp32_sum(sums[t]);
        if (lane == 0 && row < n && t0 + t < tokens) out[static_cast<std::int64_t>(t0 + t) * n + row] = from_f32<T>(y);
    }
}

// Research fused GEMV (q4_fused.cuh:10-89): lane l of a 32-lane warp owns
// byte l of every 32-byte group (columns 64g+2l, 64g+2l+1). Both products
// lo*x0 and hi*x1 are exact in fp32, so the group term RNE(lo*x0 + hi*x1) is
// the same whichever product the reference's fma contraction keeps; then
// acc = fmaf(scale, term, acc) over all padded groups in order, the 32-lane
// tree, fp16 output. One half-wave per (row, token).
__global__ __launch_bounds__(256) void q4_fused_exact(const __half* __restrict__ x,
                                                      const std::uint8_t* __restrict__ codes,
                                                      const __half* __restrict__ scales, __half* __restrict__ out,
                                                      int tokens, int rows, int k, int padded) {
    const int lane = threadIdx.x & 31;
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int token = blockIdx.y;
    float acc = 0.0f;
    if (row < rows) {
        const int groups = padded >> 6;
        const std::uint8_t* c = codes + static_cast<std::int64_t>(row) * (padded / 2);
        const __half* s = scales + static_cast<std::int64_t>(row) * groups;
        const __half* xr = x + static_cast<std::int64_t>(token) * k;
        for (int g = 0; g < groups; ++g) {
            const std::uint32_t byte = c[g * 32 + lane];
            const int col = g * 64 + 2 * lane;
            const float x0 = col < k ? __half2float(xr[col]) : 0.0f;
            const float x1 = col + 1 < k ? __half2float(xr[col + 1]) : 0.0f;
            const float lo = static_cast<float>(nibble(byte, 0)), hi = static_cast<float>(nibble(byte, 1));
            const float term = __fmaf_rn(hi, x1, __fmul_rn(lo, x0));
            acc = __fmaf_rn(__half2float(s[g]), term, acc);
        }
    }
    acc = warp32_sum(acc);
    if (lane == 0 && row < rows) out[static_cast<std::int64_t>(token) * rows + row] = from_f32<__half>(acc);
}

}  // namespace

// The expert ABI and the row decoder accept any padded >= k with padded % 128 == 0
// (flash_next_q4.cu:39,49, blocks.cu:1079); the plugin requires the minimal one.
void q4_validate(const void* codes, const void* scales, int rows, int k, int padded) {
    require(codes && scales, "null Q4 plane");
    require(rows > 0 && k > 0 && padded >= k && padded % 128 == 0, "invalid Q4 geometry");
    require(aligned(codes, 4) && aligned(scales, 2), "misaligned Q4 plane");
}

void q4_decode_launch(const void* codes, const void* scales, void* out, int row_begin, int rows, int k, int padded,
                      hipStream_t stream) {
    q4_validate(codes, scales, rows, k, padded);
    require(out && row_begin >= 0 && aligned(out, 2), "invalid Q4 decode output");
    const dim3 grid((k + 8 * 256 - 1) / (8 * 256), rows);
    require(grid.y <= 65535 * 16, "too many Q4 rows for one decode launch");
    q4_decode<<<grid, 256, 0, stream>>>(static_cast<const std::uint8_t*>(codes), static_cast<const __half*>(scales),
                                        static_cast<__half*>(out), row_begin, rows, k, padded);
}

void q4_linear_launch(const void* x, const void* codes, const void* scales, void* out, int tokens, int rows, int cols,
                      int padded, hipStream_t stream) {
    q4_validate(codes, scales, rows, cols, padded);
    require(x && out && tokens > 0 && tokens <= 64, "invalid Q4 linear operands");
    const dim3 grid((rows + 7) / 8, tokens);
    q4_linear_exact<<<grid, 256, 0, stream>>>(static_cast<const __half*>(x), static_cast<const std::uint8_t*>(codes),
                                              static_cast<const __half*>(scales), static_cast<__half*>(out), rows, cols,
                                              padded);
}

void q4_generic_launch(const void* x, const void* codes, const void* scales, void* out, int n, int k, int padded,
                       int tokens, int dtype, hipStream_t stream) {
    q4_validate(codes, scales, n, k, padded);
    require(x && out && tokens > 0 && tokens <= 4 * 65535, "invalid Q4 plugin operands");
    const dim3 grid((n + 7) / 8, (tokens + 3) / 4);
    if (dtype == kF16)
        q4_generic_exact<__half><<<grid, 256, 0, stream>>>(static_cast<const __half*>(x),
                                                           static_cast<const std::uint8_t*>(codes),
                                                           static_cast<const __half*>(scales),
                                                           static_cast<__half*>(out), n, k, padded, tokens);
    else if (dtype == kBF16)
        q4_generic_exact<__hip_bfloat16><<<grid, 256, 0, stream>>>(static_cast<const __hip_bfloat16*>(x),
                                                                   static_cast<const std::uint8_t*>(codes),
                                                                   static_cast<const __half*>(scales),
                                                                   static_cast<__hip_bfloat16*>(out), n, k, padded,
                                                                   tokens);
    else
        throw Invalid("Q4 activations must be fp16 or bf16");
}

void q4_fused_launch(const void* x, const void* codes, const void* scales, void* out, int tokens, int rows, int k,
                     int padded, int dtype, hipStream_t stream) {
    q4_validate(codes, scales, rows, k, padded);
    require(x && out && tokens > 0 && tokens <= 65535 && dtype == kF16, "invalid q4 fused GEMM geometry");
    require(static_cast<std::int64_t>(tokens) * rows < INT32_MAX, "Q4 output count exceeds int32");
    const dim3 grid((rows + 7) / 8, tokens);
    q4_fused_exact<<<grid, 256, 0, stream>>>(static_cast<const __half*>(x), static_cast<const std::uint8_t*>(codes),
                                             static_cast<const __half*>(scales), static_cast<__half*>(out), tokens,
                                             rows, k, padded);
}

}  // namespace vt

#define VT_EXPORT extern "C" __attribute__((visibility("default")))

namespace {
// The plugin ABI keeps its own thread-local error text (q4_linear.cu:10,60-61).
thread_local std::string ada_error;

template <class F>
int ada_guard(F&& body) {
    try {
        ada_error.clear();
        body();
        vt::check(hipGetLastError());
        return 0;
    } catch (const std::exception& e) {
        ada_error = e.what();
        return -1;
    }
}
}  // namespace

// ---- expert operator ABI 1 (flash_next_q4.cu:36-54): CUDA-style status codes
VT_EXPORT int venturi_q4_abi() { return 1; }

VT_EXPORT int venturi_q4_decode(const void* codes, const void* scales, void* out, int rows, int cols, int padded,
                                void* stream) {
    if (!codes || !scales || !out || rows <= 0 || cols <= 0 || padded < cols || padded % 128)
        return static_cast<int>(hipErrorInvalidValue);
    try {
        vt::q4_decode_launch(codes, scales, out, 0, rows, cols, padded, static_cast<hipStream_t>(stream));
    } catch (const std::exception&) {
        return static_cast<int>(hipErrorInvalidValue);
    }
    return static_cast<int>(hipGetLastError());
}

VT_EXPORT int venturi_q4_linear(const void* x, const void* codes, const void* scales, void* out, int tokens, int rows,
                                int cols, int padded, void* stream) {
    if (!x || !codes || !scales || !out || tokens <= 0 || tokens > 64 || rows <= 0 || cols <= 0 || padded < cols ||
        padded % 128)
        return static_cast<int>(hipErrorInvalidValue);
    try {
        vt::q4_linear_launch(x, codes, scales, out, tokens, rows, cols, padded, static_cast<hipStream_t>(stream));
    } catch (const std::exception&) {
        return static_cast<int>(hipErrorInvalidValue);
    }
    return static_cast<int>(hipGetLastError());
}

// ---- research fused Q4 GEMV (blocks.cu:1067-1076)
VT_EXPORT int venturi_q4_fused_run(const void* x, const void* codes, const void* scales, void* out, int t, int rows,
                                   int k, int padded, int dtype, void* stream) {
    return vt::guarded([&] {
        vt::q4_fused_launch(x, codes, scales, out, t, rows, k, padded, dtype, static_cast<hipStream_t>(stream));
    });
}

// ---- plugin ABI 2 (q4_linear.cu:60-88)
VT_EXPORT int venturi_ada_abi() { return 2; }
VT_EXPORT const char* venturi_ada_error() { return ada_error.c_str(); }

VT_EXPORT int venturi_q4_prepare(int n, int k, int tokens, int dtype, int requested) {
    return ada_guard([&] {
        if (n <= 0 || k <= 0 || tokens <= 0 || tokens > 4 * 65535 || dtype < 0 || dtype > 1 ||
            (requested != -1 && requested != 0))
            throw vt::Invalid("invalid Q4 dimensions, dtype, or removed route");
        int device = 0;
        vt::check(hipGetDevice(&device));
        hipDeviceProp_t props;
        vt::check(hipGetDeviceProperties(&props, device));
        if (std::string(props.gcnArchName).rfind("gfx950", 0) != 0) throw vt::Invalid("Q4 requires gfx950");
    });
}

VT_EXPORT int venturi_q4_run(const void* x, const void* codes, const void* scales, void* out, int n, int k,
                             int padded_k, int tokens, int dtype, int route, void* stream) {
    return ada_guard([&] {
        if (route != 0 || padded_k != vt::padded_k(k)) throw vt::Invalid("invalid prepared Q4 launch");
        vt::q4_generic_launch(x, codes, scales, out, n, k, padded_k, tokens, dtype, static_cast<hipStream_t>(stream));
    });
}
