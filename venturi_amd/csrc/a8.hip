// A8 activation path: per-32-group int8 activation quantization (one or two
// residual passes), RMSNorm, RMSNorm fused with quantization, and the W8A8
// decode projection in the reference's accumulation order.
//
// Workspace layout (q8_dp4a.cuh:7-13, 72-76): with G = ceil(k/32) groups and
// count = tokens*G, int8 codes [pass][token][group][32] are followed directly
// by fp32 scales [pass][token][group]; total count*36*passes bytes.
#include "a8_group.hpp"

namespace vt {

constexpr int kA8GemmMinTokens = 64;

void a8_gemm_launch(const void* workspace, const std::int8_t* codes, const __half* scales, void* out, int tokens,
                    int n, int k, int padded, int passes, int ldo, hipStream_t stream);
void a8_fast_launch(const void* workspace, const std::int8_t* codes, const __half* scales, void* out, int tokens,
                    int n, int k, int padded, int passes, hipStream_t stream);

std::uint64_t a8_bytes(int tokens, int k, int passes) {
    // Same admission as q8_dp4a.cuh:7-13.
    require(tokens > 0 && tokens <= 262140 && k > 0 && k <= INT32_MAX - 1024 && (passes == 1 || passes == 2),
            "invalid A8 geometry/profile");
    const std::uint64_t groups = (static_cast<std::uint64_t>(k) + 31) / 32;
    const std::uint64_t n = static_cast<std::uint64_t>(tokens) * groups;
    require(n <= INT32_MAX / 32, "A8 activation workspace exceeds int32");
    return n * 36 * passes;
}

namespace {

// Plain quantizer: 4 lanes per group, 8 consecutive values per lane.
__global__ __launch_bounds__(256) void a8_quantize(const __half* __restrict__ x, std::int8_t* codes,
                                                   float* scales, int tokens, int k, int groups,
                                                   int passes, bool vec) {
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const std::int64_t index = (static_cast<std::int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 2;
    const int sub = threadIdx.x & 3;
    if (index >= count) return;  // the 4 lanes of a group exit together
    const int token = static_cast<int>(index / groups);
    const int g = static_cast<int>(index % groups);
    const int col = g * 32 + sub * 8;
    const __half* src = x + static_cast<std::int64_t>(token) * k;
    float r[8];
    if (vec && col + 7 < k) {
        const uint4 w = *reinterpret_cast<const uint4*>(src + col);
        r[0] = half_lo(w.x); r[1] = half_hi(w.x); r[2] = half_lo(w.y); r[3] = half_hi(w.y);
        r[4] = half_lo(w.z); r[5] = half_hi(w.z); r[6] = half_lo(w.w); r[7] = half_hi(w.w);
    } else {
#pragma unroll
        for (int v = 0; v < 8; ++v) r[v] = col + v < k ? __half2float(src[col + v]) : 0.0f;
    }
    bool bad = false;
#pragma unroll
    for (int v = 0; v < 8; ++v) bad |= !isfinite(r[v]);
    quantize_group<8, 4>(r, bad, passes, codes + index * 32 + sub * 8, scales + index, count * 32, count,
                         sub == 0);
}

// RMS statistics of one row in the reference order (blocks.cu:31-54): 256
// sequential fmaf(v, v, s) chains over columns j, j+256, ..., then the
// two-level tree; inv = 1/sqrt(sum/k + eps) with IEEE division and square
// root. (The reference uses rsqrtf, an approximation its tests pin only by
// tolerance; this library fixes the correctly rounded form.)
// Four consecutive 16-bit values as f32, one 8-byte load (p 8-byte aligned).
template <class T>
__device__ __forceinline__ void load4_f32(const T* p, float (&v)[4]) {
    if constexpr (sizeof(T) == 2) {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        const unsigned short h[4] = {static_cast<unsigned short>(u.x), static_cast<unsigned short>(u.x >> 16),
                                     static_cast<unsigned short>(u.y), static_cast<unsigned short>(u.y >> 16)};
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = to_f32(__builtin_bit_cast(T, h[i]));
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = to_f32(p[i]);  // (rows_vec4 keeps wider types off this path)
    }
}

// Whether a row's four-value pieces can be read as 8-byte words: rows start
// 8-byte aligned when k % 4 == 0 and the base is.
template <class T>
__device__ __forceinline__ bool rows_vec4(const T* base, int k) {
    return sizeof(T) == 2 && k % 4 == 0 && (reinterpret_cast<std::uintptr_t>(base) & 7) == 0;
}

template <class T>
__device__ __forceinline__ float row_inverse_rms(const T* src, int k, float epsilon, int lane, bool vec) {
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // Unrolled so that several pieces of the row are in flight at once; each
    // chain a[v] still runs over base in ascending order.
#pragma unroll 8
    for (int base = 0; base < k; base += 256) {
        const int col = base + 4 * lane;
        if (vec && col + 3 < k) {
            float xv[4];
            load4_f32(src + col, xv);
#pragma unroll
            for (int v = 0; v < 4; ++v) a[v] = fmaf(xv[v], xv[v], a[v]);
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (col + v < k) {
                    const float x = to_f32(src[col + v]);
                    a[v] = fmaf(x, x, a[v]);
                }
        }
    }
    const float sum = __shfl(canonical_sum(a[0], a[1], a[2], a[3]), 0, 64);
    return __fdiv_rn(1.0f, sqrt_rn(__fdiv_rn(sum, static_cast<float>(k)) + epsilon));
}

// One wave per row; the normalised value is ((x * inv) * gamma) rounded once.
template <class T>
__global__ __launch_bounds__(256) void rms_norm(const T* __restrict__ x, const float* __restrict__ w,
                                                T* __restrict__ out, int tokens, int k, float epsilon) {
    const int lane = threadIdx.x & 63;
    const int token = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (token >= tokens) return;
    const T* src = x + static_cast<std::int64_t>(token) * k;
    T* dst = out + static_cast<std::int64_t>(token) * k;
    const float inv = row_inverse_rms(src, k, epsilon, lane, rows_vec4(x, k));
    for (int col = lane; col < k; col += 64) dst[col] = from_f32<T>((to_f32(src[col]) * inv) * w[col]);
}

// RMSNorm fused with A8 quantization (q8_rms_producer.cuh:8-53 for two
// passes): the quantizer sees exactly the fp16-rounded normalised values.
// One 4-wave workgroup per token: thread c runs the reference's chain c
// (fmaf over columns c, c + 256, ...), wave 0 folds the 256 chains through the
// same two-level tree as row_inverse_rms (so inv has the same bits), and the
// four waves then quantize every fourth 256-column piece; 8 lanes x 4 values
// form each group of 32.
__global__ __launch_bounds__(256) void rms_a8(const __half* __restrict__ x, const float* __restrict__ w,
                                              std::int8_t* codes, float* scales, __half* intermediate,
                                              int tokens, int k, int groups, int passes, float epsilon) {
    __shared__ float chains[256];
    __shared__ float inv_shared;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int token = blockIdx.x;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const __half* src = x + static_cast<std::int64_t>(token) * k;
    float chain = 0.0f;
#pragma unroll 4
    for (int col = tid; col < k; col += 256) {
        const float v = __half2float(src[col]);
        chain = fmaf(v, v, chain);
    }
    chains[tid] = chain;
    __syncthreads();
    if (wave == 0) {
        const float sum = canonical_sum(chains[4 * lane], chains[4 * lane + 1], chains[4 * lane + 2],
                                        chains[4 * lane + 3]);
        if (lane == 0) inv_shared = __fdiv_rn(1.0f, sqrt_rn(__fdiv_rn(sum, static_cast<float>(k)) + epsilon));
    }
    __syncthreads();
    const float inv = inv_shared;
    // Vector path: 8-byte x and intermediate pieces, 16-byte gamma pieces.
    const bool vec = rows_vec4(x, k) && (reinterpret_cast<std::uintptr_t>(w) & 15) == 0 &&
                     (!intermediate || (reinterpret_cast<std::uintptr_t>(intermediate) & 7) == 0);
    for (int base = 256 * wave; base < groups * 32; base += 1024) {
        const int col = base + 4 * lane;
        const int g = col >> 5;
        float r[4];
        bool bad = false;
        if (vec && col + 3 < k) {
            float xv[4];
            load4_f32(src + col, xv);
            const float4 wv = *reinterpret_cast<const float4*>(w + col);
            const float wa[4] = {wv.x, wv.y, wv.z, wv.w};
            unsigned short yb[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const __half y = from_f32<__half>((xv[v] * inv) * wa[v]);
                yb[v] = __half_as_ushort(y);
                r[v] = __half2float(y);
                bad |= !isfinite(r[v]);
            }
            if (intermediate)
                *reinterpret_cast<uint2*>(intermediate + static_cast<std::int64_t>(token) * k + col) =
                    make_uint2(yb[0] | (static_cast<std::uint32_t>(yb[1]) << 16),
                               yb[2] | (static_cast<std::uint32_t>(yb[3]) << 16));
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                r[v] = 0.0f;
                if (col + v < k) {
                    const __half y = from_f32<__half>((__half2float(src[col + v]) * inv) * w[col + v]);
                    if (intermediate) intermediate[static_cast<std::int64_t>(token) * k + col + v] = y;
                    r[v] = __half2float(y);
                }
                bad |= !isfinite(r[v]);
            }
        }
        const std::int64_t index = static_cast<std::int64_t>(token) * groups + min(g, groups - 1);
        // The 8 lanes of a group share g, so skipping whole groups keeps every
        // cross-lane exchange inside active lanes.
        if (g < groups)
            quantize_group<4, 8>(r, bad, passes, codes + index * 32 + (col & 31), scales + index, count * 32,
                                 count, (lane & 7) == 0);
    }
}

// One projection of a launch: resident planes, output, its row count and the
// output row stride (elements).
struct A8Item {
    const std::int8_t* codes;
    const __half* scales;
    __half* out;
    int n, stride;
};

// Up to three projections of one activation pack in one launch: workgroups
// [first[i], first[i+1]) cover item i's rows (the reference's fused
// projection, q8_fused.cuh:5-16).
struct A8Set {
    A8Item item[3];
    int first[4];
    int count;
};

// W8A8 projection in the reference order (q8_dp4a.cuh:36-70). One reference
// warp = one half-wave: lane l owns groups l, l+32, ... (< ceil(k/32));
// per group the int8 dot d is exact; sum = fmaf(f32(d), ws*as, sum) over
// passes in order; a 32-lane shfl_down tree; RNE cast to fp16. Each half-wave
// handles RR rows and TT tokens so activation words are reused RR times; a
// workgroup covers 8*RR rows of one item of the set.
template <int TT, int RR, int P>
__global__ __launch_bounds__(256) void a8_gemv(const std::int8_t* __restrict__ acodes,
                                               const float* __restrict__ ascales, const A8Set set, int tokens,
                                               int padded, int groups) {
    int item = 0;
    while (item + 1 < set.count && static_cast<int>(blockIdx.x) >= set.first[item + 1]) ++item;
    const std::int8_t* __restrict__ wcodes = set.item[item].codes;
    const __half* __restrict__ wscales = set.item[item].scales;
    __half* __restrict__ out = set.item[item].out;
    const int n = set.item[item].n, ldo = set.item[item].stride;
    const int lane = threadIdx.x & 31;
    const int half = (threadIdx.x >> 5) & 1;
    const int wave = (static_cast<int>(blockIdx.x) - set.first[item]) * 4 + (threadIdx.x >> 6);
    const int row0 = (wave * 2 + half) * RR;
    const int t0 = blockIdx.y * TT;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    float sum[TT][RR];
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int r = 0; r < RR; ++r) sum[t][r] = 0.0f;
    if (row0 < n) {
        for (int g = lane; g < groups; g += 32) {
            uint4 w0[RR], w1[RR];
            float ws[RR];
#pragma unroll
            for (int r = 0; r < RR; ++r) {
                const std::int64_t row = min(row0 + r, n - 1);
                const uint4* wp = reinterpret_cast<const uint4*>(wcodes + row * padded + g * 32);
                w0[r] = wp[0];
                w1[r] = wp[1];
                ws[r] = __half2float(wscales[row * (padded / 32) + g]);
            }
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                if (t0 + t >= tokens) break;
#pragma unroll
                for (int p = 0; p < P; ++p) {
                    const std::int64_t gi = p * count + static_cast<std::int64_t>(t0 + t) * groups + g;
                    const uint4* ap = reinterpret_cast<const uint4*>(acodes + gi * 32);
                    const uint4 a0 = ap[0], a1 = ap[1];
                    const float as = ascales[gi];
#pragma unroll
                    for (int r = 0; r < RR; ++r) {
                        int d = __builtin_amdgcn_sdot4(static_cast<int>(w0[r].x), static_cast<int>(a0.x), 0, false);
                        d = __builtin_amdgcn_sdot4(static_cast<int>(w0[r].y), static_cast<int>(a0.y), d, false);
                        d = __builtin_amdgcn_sdot4(static_cast<int>(w0[r].z), static_cast<int>(a0.z), d, false);
                        d = __builtin_amdgcn_sdot4(static_cast<int>(w0[r].w), static_cast<int>(a0.w), d, false);
                        d = __builtin_amdgcn_sdot4(static_cast<int>(w1[r].x), static_cast<int>(a1.x), d, false);
                        d = __builtin_amdgcn_sdot4(static_cast<int>(w1[r].y), static_cast<int>(a1.y), d, false);
                        d = __builtin_amdgcn_sdot4(static_cast<int>(w1[r].z), static_cast<int>(a1.z), d, false);
                        d = __builtin_amdgcn_sdot4(static_cast<int>(w1[r].w), static_cast<int>(a1.w), d, false);
                        sum[t][r] = __fmaf_rn(static_cast<float>(d), __fmul_rn(ws[r], as), sum[t][r]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int r = 0; r < RR; ++r) {
            const float y = warp32_sum(sum[t][r]);
            if (lane == 0 && row0 + r < n && t0 + t < tokens)
                out[static_cast<std::int64_t>(t0 + t) * ldo + row0 + r] = from_f32<__half>(y);
        }
}

template <int TT, int RR, int P>
void launch_a8_gemv(const std::int8_t* acodes, const float* ascales, A8Set set, int tokens, int padded, int groups,
                    hipStream_t stream) {
    constexpr int rows_per_block = 8 * RR;
    set.first[0] = 0;
    for (int i = 0; i < set.count; ++i) set.first[i + 1] = set.first[i] + (set.item[i].n + rows_per_block - 1) / rows_per_block;
    const dim3 grid(set.first[set.count], (tokens + TT - 1) / TT);
    require(grid.y <= 65535, "token tiles exceed the launch grid");
    a8_gemv<TT, RR, P><<<grid, 256, 0, stream>>>(acodes, ascales, set, tokens, padded, groups);
}

template <int P>
void dispatch_a8_gemv(const std::int8_t* acodes, const float* ascales, const A8Set& set, int tokens, int padded,
                      int groups, hipStream_t stream) {
    if (tokens == 1) launch_a8_gemv<1, 2, P>(acodes, ascales, set, tokens, padded, groups, stream);
    else if (tokens == 2) launch_a8_gemv<2, 2, P>(acodes, ascales, set, tokens, padded, groups, stream);
    else launch_a8_gemv<4, 2, P>(acodes, ascales, set, tokens, padded, groups, stream);
}

// The projections of a set in the reference's order: one SIMT launch for all
// items below 64 tokens, one matrix-core GEMM per item above (each fills the
// chip on its own).
void run_a8_set(const void* workspace, const A8Set& set, int tokens, int k, int padded, int passes,
                hipStream_t stream) {
    const int groups = (k + 31) / 32;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const auto* acodes = static_cast<const std::int8_t*>(workspace);
    const auto* ascales = reinterpret_cast<const float*>(acodes + count * 32 * passes);
    if (tokens >= kA8GemmMinTokens) {
        for (int i = 0; i < set.count; ++i)
            a8_gemm_launch(workspace, set.item[i].codes, set.item[i].scales, set.item[i].out, tokens, set.item[i].n, k,
                           padded, passes, set.item[i].stride, stream);
        return;
    }
    if (passes == 1) dispatch_a8_gemv<1>(acodes, ascales, set, tokens, padded, groups, stream);
    else dispatch_a8_gemv<2>(acodes, ascales, set, tokens, padded, groups, stream);
}

// SwiGLU of the native runtime (blocks.cu:56-86) rounded to fp16, then the
// two-pass quantizer, in one kernel (q8_producer.cuh:8-57): the bytes of
// venturi_swiglu_run followed by venturi_q8_dp4a_quantize with two passes.
// Layout and lanes as a8_quantize; `intermediate` (optional) receives the
// rounded SwiGLU values.
// `intermediate` may be gate or up itself (each element is read, then written,
// by the same lane), so those pointers carry no __restrict__.
__global__ __launch_bounds__(256) void swiglu_a8(const __half* gate, const __half* up, std::int8_t* codes,
                                                 float* scales, __half* intermediate, int tokens, int k, int groups,
                                                 bool vec) {
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    const std::int64_t index = (static_cast<std::int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 2;
    const int sub = threadIdx.x & 3;
    if (index >= count) return;  // the 4 lanes of a group exit together
    const int token = static_cast<int>(index / groups);
    const int g = static_cast<int>(index % groups);
    const int col = g * 32 + sub * 8;
    const std::int64_t row = static_cast<std::int64_t>(token) * k;
    float r[8];
    if (vec && col + 7 < k) {
        const uint4 a = *reinterpret_cast<const uint4*>(gate + row + col);
        const uint4 b = *reinterpret_cast<const uint4*>(up + row + col);
        const std::uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
        std::uint32_t hw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const __half lo = from_f32<__half>(swiglu_value(half_lo(aw[i]), half_lo(bw[i])));
            const __half hi = from_f32<__half>(swiglu_value(half_hi(aw[i]), half_hi(bw[i])));
            hw[i] = static_cast<std::uint32_t>(__half_as_ushort(lo)) | (static_cast<std::uint32_t>(__half_as_ushort(hi)) << 16);
            r[2 * i] = __half2float(lo);
            r[2 * i + 1] = __half2float(hi);
        }
        if (intermediate) *reinterpret_cast<uint4*>(intermediate + row + col) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    } else {
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            r[v] = 0.0f;
            if (col + v < k) {
                const __half h = from_f32<__half>(swiglu_value(__half2float(gate[row + col + v]), __half2float(up[row + col + v])));
                if (intermediate) intermediate[row + col + v] = h;
                r[v] = __half2float(h);
            }
        }
    }
    bool bad = false;
#pragma unroll
    for (int v = 0; v < 8; ++v) bad |= !isfinite(r[v]);
    quantize_group<8, 4>(r, bad, 2, codes + index * 32 + sub * 8, scales + index, count * 32, count, sub == 0);
}

bool overlap(const void* a, std::uint64_t an, const void* b, std::uint64_t bn) {
    const auto x = reinterpret_cast<std::uintptr_t>(a), y = reinterpret_cast<std::uintptr_t>(b);
    return x < y + bn && y < x + an;
}

}  // namespace

void a8_quantize_launch(const void* x, void* workspace, std::uint64_t available, int tokens, int k, int passes,
                        hipStream_t stream) {
    const std::uint64_t needed = a8_bytes(tokens, k, passes);
    require(x && workspace && available >= needed && aligned(workspace, 16) && aligned(x, 2),
            "invalid A8 workspace/input");
    const int groups = (k + 31) / 32;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    auto* codes = static_cast<std::int8_t*>(workspace);
    auto* scales = reinterpret_cast<float*>(codes + count * 32 * passes);
    const bool vec = (k % 8 == 0) && aligned(x, 16);
    const std::int64_t blocks = (count * 4 + 255) / 256;
    require(blocks <= INT32_MAX, "A8 grid too large");
    a8_quantize<<<static_cast<unsigned>(blocks), 256, 0, stream>>>(static_cast<const __half*>(x), codes, scales,
                                                                   tokens, k, groups, passes, vec);
}

void validate_a8_projection(const void* workspace, std::uint64_t available, const std::int8_t* codes,
                            const __half* scales, const void* out, int tokens, int n, int k, int padded, int passes) {
    const std::uint64_t needed = a8_bytes(tokens, k, passes);
    require(workspace && available >= needed && codes && scales && out && n > 0 && n <= INT32_MAX - 3 &&
                padded == padded_k(k) && static_cast<std::uint64_t>(tokens) * n < INT32_MAX &&
                aligned(workspace, 16) && aligned(codes, 16) && aligned(scales, 2) && aligned(out, 2),
            "invalid A8 projection geometry/buffers");
}

void a8_gemv_launch(const void* workspace, std::uint64_t available, const std::int8_t* codes, const __half* scales,
                    void* out, int tokens, int n, int k, int padded, int passes, hipStream_t stream) {
    validate_a8_projection(workspace, available, codes, scales, out, tokens, n, k, padded, passes);
    // Both kernels produce the reference's bytes; the matrix-core GEMM takes
    // over once a 64-token tile is filled.
    A8Set set{};
    set.item[0] = A8Item{codes, scales, static_cast<__half*>(out), n, n};
    set.count = 1;
    run_a8_set(workspace, set, tokens, k, padded, passes, stream);
}

// Reference fused-projection descriptor (ops_api.h:8-9).
struct VQFOutput {
    const std::int8_t* codes;
    const __half* scales;
    __half* out;
    int n, stride;
};
static_assert(sizeof(VQFOutput) == 32, "the reference's descriptor is 32 bytes");

void q8_fused_launch(const void* workspace, std::uint64_t available, const VQFOutput* outputs, int count, int tokens,
                     int k, int padded, int passes, hipStream_t stream) {
    // Admission of q8_fused.cuh:188-199 (the architecture check becomes gfx950).
    const std::uint64_t needed = a8_bytes(tokens, k, passes);
    require(workspace && available >= needed && outputs && (count == 2 || count == 3) && padded == padded_k(k) &&
                aligned(workspace, 16),
            "invalid fused DP4A input/geometry");
    A8Set set{};
    set.count = count;
    std::uint64_t total = 0;
    for (int i = 0; i < count; ++i) {
        const VQFOutput& p = outputs[i];
        require(p.codes && p.scales && p.out && p.n > 0 && p.n <= INT32_MAX - 16 && p.stride >= p.n &&
                    static_cast<std::uint64_t>(tokens - 1) * p.stride + p.n < INT32_MAX && aligned(p.codes, 16) &&
                    aligned(p.scales, 2) && aligned(p.out, 2),
                "invalid fused DP4A descriptor");
        total += p.n;
        set.item[i] = A8Item{p.codes, p.scales, p.out, p.n, p.stride};
    }
    require(total < INT32_MAX - 48, "fused row sum exceeds int32");
    run_a8_set(workspace, set, tokens, k, padded, passes, stream);
}

void swiglu_a8_launch(const void* gate, const void* up, void* workspace, std::uint64_t available, int tokens, int k,
                      int threads, void* intermediate, hipStream_t stream) {
    // Admission of q8_producer.cuh:62-79 (always two passes).
    const std::uint64_t needed = a8_bytes(tokens, k, 2);
    const std::uint64_t input_bytes = static_cast<std::uint64_t>(tokens) * k * 2;
    require(gate && up && workspace && available >= needed && (threads == 128 || threads == 256) &&
                aligned(workspace, 16) && aligned(gate, 2) && aligned(up, 2) && aligned(intermediate, 2) &&
                !overlap(workspace, needed, gate, input_bytes) && !overlap(workspace, needed, up, input_bytes),
            "invalid fused SwiGLU/two-pass Q8 operands");
    require(!intermediate || (!overlap(workspace, needed, intermediate, input_bytes) &&
                              (intermediate == gate || !overlap(intermediate, input_bytes, gate, input_bytes)) &&
                              (intermediate == up || !overlap(intermediate, input_bytes, up, input_bytes))),
            "invalid fused debug output overlap");
    const int groups = (k + 31) / 32;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    auto* codes = static_cast<std::int8_t*>(workspace);
    auto* scales = reinterpret_cast<float*>(codes + count * 64);
    const bool vec = k % 8 == 0 && aligned(gate, 16) && aligned(up, 16) && aligned(intermediate, 16);
    const std::int64_t blocks = (count * 4 + 255) / 256;
    require(blocks <= INT32_MAX, "A8 grid too large");
    // `threads` selects the reference's block size; the bytes do not depend on it.
    swiglu_a8<<<static_cast<unsigned>(blocks), 256, 0, stream>>>(static_cast<const __half*>(gate),
                                                                 static_cast<const __half*>(up), codes, scales,
                                                                 static_cast<__half*>(intermediate), tokens, k, groups,
                                                                 vec);
}

void rms_launch(const void* x, const float* w, void* out, int tokens, int k, int dtype, float epsilon,
                hipStream_t stream) {
    require(x && w && out && tokens > 0 && k > 0, "invalid RMSNorm operand");
    require(epsilon > 0.0f && std::isfinite(epsilon), "invalid RMSNorm epsilon");
    const dim3 grid((tokens + 3) / 4);
    if (dtype == kF16)
        rms_norm<<<grid, 256, 0, stream>>>(static_cast<const __half*>(x), w, static_cast<__half*>(out), tokens, k, epsilon);
    else if (dtype == kBF16)
        rms_norm<<<grid, 256, 0, stream>>>(static_cast<const __hip_bfloat16*>(x), w,
                                           static_cast<__hip_bfloat16*>(out), tokens, k, epsilon);
    else if (dtype == kF32)
        rms_norm<<<grid, 256, 0, stream>>>(static_cast<const float*>(x), w, static_cast<float*>(out), tokens, k, epsilon);
    else
        throw Invalid("unsupported scalar type");
}

void rms_a8_launch(const void* x, const float* w, void* workspace, std::uint64_t available, int tokens, int k,
                   float epsilon, int passes, void* intermediate, hipStream_t stream) {
    const std::uint64_t needed = a8_bytes(tokens, k, passes);
    const std::uint64_t xb = static_cast<std::uint64_t>(tokens) * k * 2, wb = static_cast<std::uint64_t>(k) * 4;
    require(x && w && workspace && available >= needed && epsilon > 0.0f && std::isfinite(epsilon) &&
                aligned(x, 2) && aligned(w, 4) && aligned(workspace, 16) && aligned(intermediate, 2) &&
                !overlap(workspace, needed, x, xb) && !overlap(workspace, needed, w, wb) &&
                (!intermediate || (!overlap(intermediate, xb, x, xb) && !overlap(intermediate, xb, w, wb) &&
                                   !overlap(intermediate, xb, workspace, needed))),
            "invalid RMS/A8 operands");
    const int groups = (k + 31) / 32;
    const std::int64_t count = static_cast<std::int64_t>(tokens) * groups;
    auto* codes = static_cast<std::int8_t*>(workspace);
    auto* scales = reinterpret_cast<float*>(codes + count * 32 * passes);
    rms_a8<<<tokens, 256, 0, stream>>>(static_cast<const __half*>(x), w, codes, scales,
                                       static_cast<__half*>(intermediate), tokens, k, groups, passes, epsilon);
}

}  // namespace vt

#define VT_EXPORT extern "C" __attribute__((visibility("default")))

// Reference: q8_dp4a.cuh:90-92. Returns 0 on invalid geometry.
VT_EXPORT std::uint64_t venturi_q8_dp4a_bytes(int tokens, int k, int passes) {
    std::uint64_t result = 0;
    if (!vt::host_guarded([&] { result = vt::a8_bytes(tokens, k, passes); })) return 0;
    return result;
}

// Reference: q8_dp4a.cuh:93-101.
VT_EXPORT int venturi_q8_dp4a_quantize(const void* x, void* workspace, std::uint64_t available, int tokens, int k,
                                       int passes, void* stream) {
    return vt::guarded([&] {
        vt::a8_quantize_launch(x, workspace, available, tokens, k, passes, static_cast<hipStream_t>(stream));
    });
}

// Reference: q8_dp4a.cuh:102-109.
VT_EXPORT int venturi_q8_dp4a_run(const void* workspace, std::uint64_t available, const std::int8_t* codes,
                                  const __half* scales, void* out, int tokens, int n, int k, int padded, int passes,
                                  void* stream) {
    return vt::guarded([&] {
        vt::a8_gemv_launch(workspace, available, codes, scales, out, tokens, n, k, padded, passes,
                           static_cast<hipStream_t>(stream));
    });
}

// Extension: the same W8A8 projection on matrix cores with the groups summed
// in natural order (exact int32 group dots, fp32 association differs from the
// reference's lane-slot tree); same arguments and workspace as
// venturi_q8_dp4a_run.
VT_EXPORT int venturi_q8_a8_gemm_run(const void* workspace, std::uint64_t available, const std::int8_t* codes,
                                     const __half* scales, void* out, int tokens, int n, int k, int padded,
                                     int passes, void* stream) {
    return vt::guarded([&] {
        vt::validate_a8_projection(workspace, available, codes, scales, out, tokens, n, k, padded, passes);
        vt::a8_fast_launch(workspace, codes, scales, out, tokens, n, k, padded, passes,
                           static_cast<hipStream_t>(stream));
    });
}

// Reference: blocks.cu:727-740.
VT_EXPORT int venturi_rms_run(const void* x, const float* w, void* out, int tokens, int features, int dtype,
                              float epsilon, void* stream) {
    return vt::guarded([&] {
        vt::rms_launch(x, w, out, tokens, features, dtype, epsilon, static_cast<hipStream_t>(stream));
    });
}

// Reference: q8_rms_producer.cuh:67-84 (two passes; `chunk` is validated
// for ABI compatibility and does not change the bytes produced).
VT_EXPORT int venturi_rms_q8_quantize(const void* x, const float* w, void* workspace, std::uint64_t available,
                                      int tokens, int k, float epsilon, int chunk, void* intermediate,
                                      void* stream) {
    return vt::guarded([&] {
        vt::require(chunk == 8 || chunk == 32 || chunk == 128, "invalid RMS/A8 chunk");
        vt::rms_a8_launch(x, w, workspace, available, tokens, k, epsilon, 2, intermediate,
                          static_cast<hipStream_t>(stream));
    });
}

// Extension: the same fused producer with an explicit pass count (1 or 2).
VT_EXPORT int venturi_rms_q8_quantize_passes(const void* x, const float* w, void* workspace,
                                             std::uint64_t available, int tokens, int k, float epsilon, int passes,
                                             void* intermediate, void* stream) {
    return vt::guarded([&] {
        vt::rms_a8_launch(x, w, workspace, available, tokens, k, epsilon, passes, intermediate,
                          static_cast<hipStream_t>(stream));
    });
}

// Reference fused projection (ops_api.h:61, q8_fused.cuh:186-205): two or three
// Q8 matrices against one A8 activation pack, each output written with its
// own row stride; bytes equal venturi_q8_dp4a_run per matrix.
VT_EXPORT int venturi_q8_fused_run(const void* workspace, std::uint64_t available, const vt::VQFOutput* outputs,
                                   int count, int tokens, int k, int padded, int passes, void* stream) {
    return vt::guarded([&] {
        vt::q8_fused_launch(workspace, available, outputs, count, tokens, k, padded, passes,
                            static_cast<hipStream_t>(stream));
    });
}

// Reference SwiGLU -> two-pass A8 producer (ops_api.h:99, q8_producer.cuh:60-82).
VT_EXPORT int venturi_swiglu_q8_quantize(const void* gate, const void* up, void* workspace, std::uint64_t available,
                                         int tokens, int k, int threads, void* intermediate_debug, void* stream) {
    return vt::guarded([&] {
        vt::swiglu_a8_launch(gate, up, workspace, available, tokens, k, threads, intermediate_debug,
                             static_cast<hipStream_t>(stream));
    });
}
