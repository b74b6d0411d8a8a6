// Dense projections through hipBLASLt. W*A16 (q4/q5/q6): the reference's ChunkedDense path
// (row_codec_dispatch.cuh:41-48 admits it for q4/q5/q6_g64; Model::project
// runs it as row_dense_project, qwen_runtime.cuh:348-364) for gfx950.
//
// For each chunk of weight rows: decode the rows to the contract's fp16
// weights fp16(q * scale) (row_decode_launch, the kernel of
// venturi_row_dequant_rows) into a shadow inside the caller's workspace, then
// one hipBLASLt GEMM (fp16 operands, fp32 accumulation, fp16 output) writes
// the chunk's columns of out in place (ldd = n), where the reference GEMMs
// into a staging chunk and copies it over with cudaMemcpy2DAsync.
//
// Chunking: a matrix whose fp16 shadow is at most 192 MiB is decoded whole
// (one GEMM keeps the whole grid of output tiles). Larger matrices run in
// chunks of whole 1024-row blocks within 80 MiB (8192 rows at K = 5120): the
// GEMM re-reads its weight chunk once per row of token tiles, and a chunk of
// that size stays in the 256 MB Infinity Cache between those reads. Measured
// on config-2 gate+up (34816 x 5120) at 2048 tokens: 702 us whole, 598 us in
// 8192-row chunks, 614 in 7168; 8704- and 17408-row chunks took 760 and
// 884 us (hipBLASLt's kernels for those row counts launch fewer workgroups
// than the chip has CUs). A smaller workspace gives smaller chunks
// (multiples of 16 rows).
//
// hipBLASLt state: one handle per device and one (descriptor, layouts,
// algorithm) entry per (device, dtype, tokens, rows, k, n, workspace share),
// made on first use under a mutex and kept for the life of the process (the
// bridge's share is bucketed to 17 sizes, so the cache stays bounded by the
// shapes a process runs). That first call per key allocates the handle's
// resources and queries the heuristic, so it must not run under graph
// capture; later calls with the same key make no allocation and are
// capturable.
#include "common.hpp"

#include "../../include/venturi_ops.h"

#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

namespace vt {

void row_decode_launch(const void* codes, const void* high, const void* scales, const std::int64_t* ids, void* out,
                       int row_begin, int rows, int k, int padded, int bits, hipStream_t stream);
void q8_split_launch(const std::int8_t* codes, const __half* scales, void* shadow, int row0, int rows, int k,
                     int padded, hipStream_t stream);
void q8_dup_launch(const void* x, void* x2, int tokens, int k, hipStream_t stream);

namespace {

constexpr std::uint64_t kBlasBytes = 32ull << 20;    // hipBLASLt's share, at the start of the workspace
constexpr std::uint64_t kWholeBytes = 192ull << 20;  // shadows up to this size are decoded whole
constexpr std::uint64_t kChunkBytes = 80ull << 20;   // else chunks of 1024-row blocks within this size

void blas(hipblasStatus_t status, const char* what) {
    if (status != HIPBLAS_STATUS_SUCCESS)
        throw std::runtime_error(std::string("hipBLASLt ") + what + " failed (status " + std::to_string(status) + ")");
}

int policy_rows(int n, int k) {
    if (2ull * n * k <= kWholeBytes) return n;
    const std::uint64_t blocks = std::max<std::uint64_t>(1, kChunkBytes / (2048ull * k));
    return static_cast<int>(std::min<std::uint64_t>(n, blocks * 1024));
}

void check_geometry(int tokens, int n, int k) {
    require(tokens > 0 && n > 0 && k > 0, "invalid dense projection geometry");
    require(k % 8 == 0 && n % 8 == 0, "the dense route needs k % 8 == 0 and n % 8 == 0");
}

struct Gemm {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

struct DeviceBlas {
    hipblasLtHandle_t handle = nullptr;
    std::map<std::tuple<int, int, int, int, int, std::uint64_t>, Gemm> gemms;
};

hipDataType blas_type(int dtype) {
    require(dtype == kF16 || dtype == kBF16 || dtype == kF32, "unsupported scalar type");
    return dtype == kF16 ? HIP_R_16F : dtype == kBF16 ? HIP_R_16BF : HIP_R_32F;
}

std::mutex blas_mutex;

// D (rows x tokens, column-major, ldd = n) = A^T B: A is the shadow chunk
// (k x rows column-major, i.e. [rows][k] row-major), B is x (k x tokens
// column-major, i.e. [tokens][k] row-major); D is out[t][begin + j].
std::pair<hipblasLtHandle_t, const Gemm*> gemm_for(int tokens, int rows, int k, int n, int dtype = kF16,
                                                   std::uint64_t limit = kBlasBytes) {
    int device = 0;
    check(hipGetDevice(&device));
    const hipDataType type = blas_type(dtype);
    std::lock_guard<std::mutex> lock(blas_mutex);
    static std::map<int, DeviceBlas> devices;
    DeviceBlas& dev = devices[device];
    if (!dev.handle) blas(hipblasLtCreate(&dev.handle), "handle creation");
    const auto key = std::make_tuple(dtype, tokens, rows, k, n, limit);
    auto found = dev.gemms.find(key);
    if (found != dev.gemms.end()) return {dev.handle, &found->second};

    Gemm g;
    blas(hipblasLtMatmulDescCreate(&g.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "descriptor creation");
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    blas(hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)), "transpose A");
    blas(hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)), "transpose B");
    blas(hipblasLtMatrixLayoutCreate(&g.a, type, k, rows, k), "layout A");
    blas(hipblasLtMatrixLayoutCreate(&g.b, type, k, tokens, k), "layout B");
    blas(hipblasLtMatrixLayoutCreate(&g.d, type, rows, tokens, n), "layout D");
    hipblasLtMatmulPreference_t pref = nullptr;
    blas(hipblasLtMatmulPreferenceCreate(&pref), "preference creation");
    blas(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &limit, sizeof(limit)),
         "workspace preference");
    hipblasLtMatmulHeuristicResult_t result{};
    int count = 0;
    const hipblasStatus_t found_algo =
        hipblasLtMatmulAlgoGetHeuristic(dev.handle, g.desc, g.a, g.b, g.d, g.d, pref, 1, &result, &count);
    hipblasLtMatmulPreferenceDestroy(pref);
    blas(found_algo, "algorithm search");
    require(count > 0 && result.state == HIPBLAS_STATUS_SUCCESS, "hipBLASLt has no algorithm for this dense GEMM");
    g.algo = result.algo;
    auto placed = dev.gemms.emplace(key, g).first;
    return {dev.handle, &placed->second};
}

void dense_run(const void* x, const void* codes, const void* high, const void* scales, void* out, int tokens, int n,
               int k, int padded, int bits, int dtype, void* workspace, std::uint64_t bytes, hipStream_t stream) {
    require(dtype == kF16, "the dense W*A16 route takes fp16 activations");
    require(bits >= 4 && bits <= 6, "row codecs are 4, 5 or 6 bits");
    check_geometry(tokens, n, k);
    require(x && out && workspace, "null dense projection operand");
    require(aligned(x, 16) && aligned(out, 16) && aligned(workspace, 256),
            "the dense route needs 16-byte x and out and a 256-byte aligned workspace");
    const std::uint64_t shadow_bytes = bytes > kBlasBytes ? bytes - kBlasBytes : 0;
    int rows = policy_rows(n, k);
    if (shadow_bytes / (2ull * k) < static_cast<std::uint64_t>(rows))
        rows = static_cast<int>(shadow_bytes / (2ull * k)) / 16 * 16;
    require(rows > 0, "the workspace holds no 16-row chunk of the fp16 shadow (see venturi_row_dense_workspace_bytes)");
    auto* shadow = static_cast<unsigned char*>(workspace) + kBlasBytes;
    const float alpha = 1.0f, beta = 0.0f;
    for (int begin = 0; begin < n; begin += rows) {
        const int r = std::min(rows, n - begin);
        row_decode_launch(codes, high, scales, nullptr, shadow, begin, r, k, padded, bits, stream);
        const auto [handle, g] = gemm_for(tokens, r, k, n);
        __half* d = static_cast<__half*>(out) + begin;
        blas(hipblasLtMatmul(handle, g->desc, &alpha, shadow, g->a, x, g->b, &beta, d, g->d, d, g->d, &g->algo,
                             workspace, kBlasBytes, stream),
             "GEMM launch");
    }
}

// The Q8 form: the W8A16 contract scales each exact group dot, so the
// decoded weights must be q*s exactly; the shadow holds each row as its two
// fp16 terms [hi | lo] (q8_split) and the activations are doubled to [x | x],
// so one GEMM over 2k columns sums x*hi + x*lo, every product exact, in fp32.
// Chunks: whole matrices up to 8192 rows, else 8192-row chunks (config-2
// gate+up, K = 2 x 5120: 1024 us in 8192-row chunks against 1149-1294 in
// 4096- to 6144-row ones and 1170 whole; down, K = 2 x 17408, is faster whole).
constexpr int kQ8ChunkRows = 8192;

std::uint64_t q8_x2_bytes(int tokens, int k) { return (4ull * tokens * k + 255) / 256 * 256; }

void q8_dense_run(const void* x, const std::int8_t* codes, const __half* scales, void* out, int tokens, int n, int k,
                  int padded, int dtype, void* workspace, std::uint64_t bytes, hipStream_t stream) {
    require(dtype == kF16, "the dense Q8 route takes fp16 activations");
    check_geometry(tokens, n, k);
    require(tokens <= 65535, "the dense Q8 route takes at most 65535 tokens");
    require(x && codes && scales && out && workspace, "null dense projection operand");
    require(padded == padded_k(k), "invalid Q8 geometry");
    require(aligned(x, 16) && aligned(out, 16) && aligned(workspace, 256) && aligned(codes, 8),
            "the dense route needs 16-byte x and out, 8-byte codes and a 256-byte aligned workspace");
    const std::uint64_t x2 = q8_x2_bytes(tokens, k);
    const std::uint64_t shadow_bytes = bytes > kBlasBytes + x2 ? bytes - kBlasBytes - x2 : 0;
    int rows = std::min(n, kQ8ChunkRows);
    if (shadow_bytes / (4ull * k) < static_cast<std::uint64_t>(rows))
        rows = static_cast<int>(shadow_bytes / (4ull * k)) / 16 * 16;
    require(rows > 0, "the workspace holds no 16-row chunk of the fp16 shadow (see venturi_q8_dense_workspace_bytes)");
    auto* xd = static_cast<unsigned char*>(workspace) + kBlasBytes;
    auto* shadow = xd + x2;
    q8_dup_launch(x, xd, tokens, k, stream);
    const float alpha = 1.0f, beta = 0.0f;
    for (int begin = 0; begin < n; begin += rows) {
        const int r = std::min(rows, n - begin);
        q8_split_launch(codes, scales, shadow, begin, r, k, padded, stream);
        const auto [handle, g] = gemm_for(tokens, r, 2 * k, n);
        __half* d = static_cast<__half*>(out) + begin;
        blas(hipblasLtMatmul(handle, g->desc, &alpha, shadow, g->a, xd, g->b, &beta, d, g->d, d, g->d, &g->algo,
                             workspace, kBlasBytes, stream),
             "GEMM launch");
    }
}

// The reference's dense bridge (venturi_dense_create/run/destroy,
// blocks.cu:674-713): out[t][n] = x[t][k] w[n][k]^T in the plan's dtype
// (0 fp16, 1 bf16, 2 fp32) with fp32 arithmetic, the caller's buffer as the
// GEMM workspace. hipBLASLt in cuBLAS's place; the plan holds only its dtype
// (the per-device handle and per-shape algorithms are shared, see gemm_for).
struct DenseLinear {
    int dtype;
};

// The workspace share handed to hipBLASLt for a caller's buffer of `bytes`:
// at most 32 MiB, rounded down to a power of two (0 below 1 KiB). The
// per-shape algorithm cache is keyed on it, so callers that size their buffer
// differently share a few entries (at most 16 per shape) instead of adding
// one, and one heuristic query, per distinct size.
std::uint64_t workspace_bucket(std::uint64_t bytes) {
    if (bytes < 1024) return 0;
    std::uint64_t bucket = 1024;
    while (bucket * 2 <= std::min<std::uint64_t>(bytes, kBlasBytes)) bucket *= 2;
    return bucket;
}

void dense_linear_run(const DenseLinear* p, const void* x, const void* w, void* out, int tokens, int n, int k,
                      void* workspace, std::uint64_t bytes, hipStream_t stream) {
    require(p && x && w && out && workspace, "null Linear operand");
    require(tokens > 0 && n > 0, "invalid shape");
    require(k > 0, "invalid K");
    // hipBLASLt's kernels read operands in 16-byte vectors; the runtime's own
    // buffers (allocations and whole-row offsets of them) meet this.
    require(aligned(x, 16) && aligned(w, 16) && aligned(out, 16) && aligned(workspace, 16),
            "the dense bridge needs 16-byte aligned x, w, out and workspace");
    const std::uint64_t share = workspace_bucket(bytes);
    const auto [handle, g] = gemm_for(tokens, n, k, n, p->dtype, share);
    const float alpha = 1.0f, beta = 0.0f;
    blas(hipblasLtMatmul(handle, g->desc, &alpha, w, g->a, x, g->b, &beta, out, g->d, out, g->d, &g->algo, workspace,
                         share, stream),
         "GEMM launch");
}

}  // namespace
}  // namespace vt

#define VT_EXPORT extern "C" __attribute__((visibility("default")))

VT_EXPORT void* venturi_dense_create(int dtype) {
    vt::DenseLinear* plan = nullptr;
    vt::host_guarded([&] {
        (void)vt::blas_type(dtype);
        plan = new vt::DenseLinear{dtype};
    });
    return plan;
}

VT_EXPORT void venturi_dense_destroy(void* opaque) { delete static_cast<vt::DenseLinear*>(opaque); }

VT_EXPORT int venturi_dense_run(void* opaque, const void* x, const void* w, void* out, int tokens, int n, int k,
                                void* workspace, size_t workspace_bytes, void* stream) {
    return vt::guarded([&] {
        vt::dense_linear_run(static_cast<const vt::DenseLinear*>(opaque), x, w, out, tokens, n, k, workspace,
                             workspace_bytes, static_cast<hipStream_t>(stream));
    });
}

VT_EXPORT uint64_t venturi_q8_dense_workspace_bytes(int tokens, int n, int k) {
    std::uint64_t bytes = 0;
    vt::host_guarded([&] {
        vt::check_geometry(tokens, n, k);
        vt::require(tokens <= 65535, "the dense Q8 route takes at most 65535 tokens");
        bytes = vt::kBlasBytes + vt::q8_x2_bytes(tokens, k) + 4ull * std::min(n, vt::kQ8ChunkRows) * k;
    });
    return bytes;
}

VT_EXPORT int venturi_q8_dense_run(const void* x, const int8_t* codes, const void* scales, void* out, int tokens,
                                   int n, int k, int padded, int dtype, void* workspace, uint64_t workspace_bytes,
                                   void* stream) {
    return vt::guarded([&] {
        vt::q8_dense_run(x, codes, static_cast<const __half*>(scales), out, tokens, n, k, padded, dtype, workspace,
                         workspace_bytes, static_cast<hipStream_t>(stream));
    });
}

VT_EXPORT uint64_t venturi_row_dense_workspace_bytes(int tokens, int n, int k) {
    std::uint64_t bytes = 0;
    vt::host_guarded([&] {
        vt::check_geometry(tokens, n, k);
        bytes = vt::kBlasBytes + 2ull * vt::policy_rows(n, k) * k;
    });
    return bytes;
}

VT_EXPORT int venturi_row_dense_run(const void* x, const void* codes, const void* high, const void* scales, void* out,
                                    int tokens, int n, int k, int padded, int bits, int dtype, void* workspace,
                                    uint64_t workspace_bytes, void* stream) {
    return vt::guarded([&] {
        vt::dense_run(x, codes, high, scales, out, tokens, n, k, padded, bits, dtype, workspace, workspace_bytes,
                      static_cast<hipStream_t>(stream));
    });
}
