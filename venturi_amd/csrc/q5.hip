// Q5 / Q6 (q5_g64_fp16, q6_g64_fp16) row codecs on gfx950: fp16 row decode
// for 4-, 5- and 6-bit rows, and the reference's W5A16 expert-style GEMV.
//
// Layout (weights.py:175-190, weight_dequant.cuh:1-9): codes uint8
// [n][padded/2] hold the low four bits (column 2j in the low nibble of byte
// j); a high plane uint8 [n][padded*hb/8] holds the remaining hb = bits-4
// bits of every column as an LSB-first bit stream (column c's bits start at
// bit c*hb of the row); scales fp16 [n][padded/64]. q is the bits-wide two's
// complement of (low | high << 4); a weight is fp16(q * scale), one RNE
// rounding of the exact product.
#include "common.hpp"

namespace vt {
namespace {

// Eight consecutive columns [col, col+8) of one row, col % 8 == 0, as fp16
// bit patterns. HB = bits - 4 (0, 1 or 2).
template <int HB>
__device__ __forceinline__ void decode_octet(const std::uint8_t* __restrict__ codes,
                                             const std::uint8_t* __restrict__ high,
                                             const __half* __restrict__ scales, std::int64_t row, int col,
                                             int padded, unsigned short (&h)[8]) {
    const std::uint32_t word = *reinterpret_cast<const std::uint32_t*>(codes + row * (padded / 2) + col / 2);
    std::uint32_t hi = 0;
    if constexpr (HB == 1) hi = high[row * (padded / 8) + col / 8];
    if constexpr (HB == 2) hi = *reinterpret_cast<const unsigned short*>(high + row * (padded / 4) + col / 4);
    const float s = __half2float(scales[row * (padded / 64) + col / 64]);
    constexpr int bits = 4 + HB, sign = 1 << (bits - 1);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        int raw = static_cast<int>((word >> (4 * j)) & 15u);
        if constexpr (HB > 0) raw |= static_cast<int>((hi >> (HB * j)) & ((1u << HB) - 1u)) << 4;
        const int q = (raw ^ sign) - sign;
        h[j] = __half_as_ushort(from_f32<__half>(static_cast<float>(q) * s));
    }
}

// Row decode: workgroup (x, y) writes columns [2048 x, 2048 x + 2048) of
// output row y = source row ids[y] (indexed) or row_begin + y; output rows are
// contiguous with ld = k. Padding columns (>= k) are never written.
template <int HB, bool INDEXED>
__global__ __launch_bounds__(256) void row_decode(const std::uint8_t* __restrict__ codes,
                                                  const std::uint8_t* __restrict__ high,
                                                  const __half* __restrict__ scales,
                                                  const std::int64_t* __restrict__ ids, __half* __restrict__ out,
                                                  int row_begin, int rows, int k, int padded) {
    const int local = blockIdx.y;
    const int col = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (local >= rows || col >= k) return;
    const std::int64_t row = INDEXED ? ids[local] : static_cast<std::int64_t>(row_begin) + local;
    unsigned short h[8];
    decode_octet<HB>(codes, high, scales, row, col, padded, h);
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

// W5A16 GEMV (flash_next_q5.cu:26-38): for output (t, row) lane l of a
// 32-lane reference warp accumulates sum = fmaf(w(col), x[col], sum) over
// col = l, l+32, ... < cols with w = fp16(q*scale), then the shfl_down
// 16/8/4/2/1 tree; fp16 output. (The reference writes sum += w*x, which nvcc
// contracts to that fmaf.) One half-wave per (row, token).
__global__ __launch_bounds__(256) void q5_linear_exact(const __half* __restrict__ x,
                                                       const std::uint8_t* __restrict__ codes,
                                                       const std::uint8_t* __restrict__ high,
                                                       const __half* __restrict__ scales, __half* __restrict__ out,
                                                       int rows, int cols, int padded) {
    const int lane = threadIdx.x & 31;
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int token = blockIdx.y;
    float sum = 0.0f;
    if (row < rows) {
        const std::uint8_t* c = codes + static_cast<std::int64_t>(row) * (padded / 2);
        const std::uint8_t* hp = high + static_cast<std::int64_t>(row) * (padded / 8);
        const __half* s = scales + static_cast<std::int64_t>(row) * (padded / 64);
        const __half* xr = x + static_cast<std::int64_t>(token) * cols;
        for (int col = lane; col < cols; col += 32) {
            const int raw = static_cast<int>((c[col >> 1] >> (4 * (col & 1))) & 15) |
                            (static_cast<int>((hp[col >> 3] >> (col & 7)) & 1) << 4);
            const int q = (raw ^ 16) - 16;
            const float w = __half2float(from_f32<__half>(static_cast<float>(q) * __half2float(s[col >> 6])));
            sum = fmaf(w, __half2float(xr[col]), sum);
        }
    }
    sum = warp32_sum(sum);
    if (lane == 0 && row < rows) out[static_cast<std::int64_t>(token) * rows + row] = from_f32<__half>(sum);
}

}  // namespace

// Any padded >= k with padded % 128 == 0 (blocks.cu:1079, flash_next_q5.cu:41-42).
void row_decode_launch(const void* codes, const void* high, const void* scales, const std::int64_t* ids, void* out,
                       int row_begin, int rows, int k, int padded, int bits, hipStream_t stream) {
    require(bits == 4 || bits == 5 || bits == 6, "row codecs are 4, 5 or 6 bits");
    require(codes && scales && out && (bits == 4 || high), "null row-codec plane");
    require(rows > 0 && k > 0 && padded >= k && padded % 128 == 0 && row_begin >= 0, "invalid row-codec geometry");
    require(aligned(codes, 4) && aligned(high, 2) && aligned(scales, 2) && aligned(out, 2), "misaligned row-codec plane");
    const dim3 grid((k + 8 * 256 - 1) / (8 * 256), rows);
    require(grid.y <= 65535 * 16, "too many rows for one decode launch");
    const auto* c = static_cast<const std::uint8_t*>(codes);
    const auto* h = static_cast<const std::uint8_t*>(high);
    const auto* s = static_cast<const __half*>(scales);
    auto* o = static_cast<__half*>(out);
#define VT_ROW_DECODE(HB)                                                                                 \
    do {                                                                                                  \
        if (ids) row_decode<HB, true><<<grid, 256, 0, stream>>>(c, h, s, ids, o, 0, rows, k, padded);      \
        else row_decode<HB, false><<<grid, 256, 0, stream>>>(c, h, s, nullptr, o, row_begin, rows, k, padded); \
    } while (0)
    if (bits == 4) VT_ROW_DECODE(0);
    else if (bits == 5) VT_ROW_DECODE(1);
    else VT_ROW_DECODE(2);
#undef VT_ROW_DECODE
}

void q5_linear_launch(const void* x, const void* codes, const void* high, const void* scales, void* out, int tokens,
                      int rows, int cols, int padded, hipStream_t stream) {
    require(x && codes && high && scales && out && tokens > 0 && tokens <= 64 && rows > 0 && cols > 0 &&
                padded >= cols && padded % 128 == 0,
            "invalid Q5 linear operands");
    require(aligned(x, 2) && aligned(scales, 2) && aligned(out, 2), "misaligned Q5 operand");
    const dim3 grid((rows + 7) / 8, tokens);
    q5_linear_exact<<<grid, 256, 0, stream>>>(static_cast<const __half*>(x), static_cast<const std::uint8_t*>(codes),
                                              static_cast<const std::uint8_t*>(high),
                                              static_cast<const __half*>(scales), static_cast<__half*>(out), rows,
                                              cols, padded);
}

}  // namespace vt

#define VT_EXPORT extern "C" __attribute__((visibility("default")))

// ---- row-codec decode (blocks.cu:1077-1096): contiguous rows, or rows by id.
// `ids` are int64 row indices of the planes; every id must name a row that
// exists (the signature carries no row count, as in the reference).
VT_EXPORT int venturi_row_dequant_rows(const void* codes, const void* high, const void* scales, void* out, int row,
                                       int rows, int k, int padded, int bits, void* stream) {
    return vt::guarded([&] {
        vt::row_decode_launch(codes, high, scales, nullptr, out, row, rows, k, padded, bits,
                              static_cast<hipStream_t>(stream));
    });
}

VT_EXPORT int venturi_row_dequant_indexed(const void* codes, const void* high, const void* scales,
                                          const std::int64_t* ids, void* out, int count, int k, int padded, int bits,
                                          void* stream) {
    return vt::guarded([&] {
        vt::require(ids && vt::aligned(ids, 8), "null or misaligned row ids");
        vt::row_decode_launch(codes, high, scales, ids, out, 0, count, k, padded, bits,
                              static_cast<hipStream_t>(stream));
    });
}

// ---- W5A16 operator ABI 1 (flash_next_q5.cu:40-64): CUDA-style status codes.
VT_EXPORT int venturi_q5_abi() { return 1; }

VT_EXPORT int venturi_q5_decode(const void* codes, const void* high, const void* scales, void* out, int rows,
                                int cols, int padded, void* stream) {
    if (!codes || !high || !scales || !out || rows <= 0 || cols <= 0 || padded < cols || padded % 128)
        return static_cast<int>(hipErrorInvalidValue);
    try {
        vt::row_decode_launch(codes, high, scales, nullptr, out, 0, rows, cols, padded, 5,
                              static_cast<hipStream_t>(stream));
    } catch (const std::exception&) {
        return static_cast<int>(hipErrorInvalidValue);
    }
    return static_cast<int>(hipGetLastError());
}

VT_EXPORT int venturi_q5_linear(const void* x, const void* codes, const void* high, const void* scales, void* out,
                                int tokens, int rows, int cols, int padded, void* stream) {
    if (!x || !codes || !high || !scales || !out || tokens <= 0 || tokens > 64 || rows <= 0 || cols <= 0 ||
        padded < cols || padded % 128)
        return static_cast<int>(hipErrorInvalidValue);
    try {
        vt::q5_linear_launch(x, codes, high, scales, out, tokens, rows, cols, padded,
                             static_cast<hipStream_t>(stream));
    } catch (const std::exception&) {
        return static_cast<int>(hipErrorInvalidValue);
    }
    return static_cast<int>(hipGetLastError());
}
