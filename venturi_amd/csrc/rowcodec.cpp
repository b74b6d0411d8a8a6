// The native runtime's QuantLinear plan table and per-matrix projection
// dispatch: rowcodec::prepare (row_codec_dispatch.cuh:6-64) and the
// per-matrix part of Model::project (qwen_runtime.cuh:348-390), restated over
// this library's kernels for gfx950. Host code only: admission is decided
// once at load from (bits, group, precision, dtype, implementation), never
// from shapes, and projection calls the entry points below.
#include "common.hpp"

#include "../../include/venturi_ops.h"

namespace vt {
namespace {

enum Precision : int { kWxA16 = 0, kWxA8 = 1, kWxA8Residual = 2 };
enum Implementation : int { kAuto = 0, kDequant = 1, kFusedResearch = 2 };
enum Path : int { kDirect = 0, kChunkedDense = 1, kQuantized = 2 };

// ChunkedDense plans from this many tokens run the decoded-shadow GEMM
// (venturi_row_dense_run) when the caller's workspace holds it. Its workspace
// is one fixed buffer, as the reference runtime's dequant buffer is: the
// 32 MiB hipBLASLt share plus 192 MiB of shadow, which holds any matrix the
// dense route decodes whole and every chunk it cuts larger ones into.
constexpr int kDenseTokens = 1024;
constexpr std::uint64_t kDenseMinBytes = 32ull << 20;
constexpr std::uint64_t kDenseBytes = kDenseMinBytes + (192ull << 20);

// rowcodec::prepare's table with the architecture gate replaced by gfx950
// (the only target of this library):
//  * q8_g32: Auto only; WxA16 -> Direct (fp16 or bf16); WxA8 and
//    WxA8Residual -> Quantized (fp16 only), one or two activation passes;
//  * q4/q5/q6_g64, fp16 only, WxA16: Auto or Dequant -> ChunkedDense (the
//    W*A16 contract, fp16(q*scale) weights); FusedResearch -> Direct for q4
//    (the research fused GEMV). The reference also admits q5 FusedResearch
//    (venturi_q5_fused_run, on SM70 and SM89) and q5 A8 (SM70 only); this
//    library builds neither research kernel, so both are refused with a
//    message rather than routed elsewhere.
VRCPlan admit(int bits, int group, int precision, int dtype, int implementation) {
    require(dtype == kF16 || dtype == kBF16, "row-codec plans take fp16 or bf16 activations");
    require(precision >= kWxA16 && precision <= kWxA8Residual, "unknown row-codec precision");
    require(implementation >= kAuto && implementation <= kFusedResearch, "unknown row-codec implementation");
    VRCPlan plan{};
    plan.bits = bits;
    plan.group = group;
    plan.precision = precision;
    plan.dtype = dtype;
    plan.implementation = implementation;
    if (bits == 8 && group == 32) {
        require(implementation == kAuto, "q8_g32 plans admit the Auto implementation only");
        require(precision == kWxA16 || dtype == kF16, "A8 plans take fp16 activations");
        plan.path = precision == kWxA16 ? kDirect : kQuantized;
        plan.passes = precision == kWxA16 ? 0 : precision == kWxA8 ? 1 : 2;
        return plan;
    }
    require(group == 64 && bits >= 4 && bits <= 6, "no row-codec plan for this (bits, group)");
    require(dtype == kF16, "q4/q5/q6 plans take fp16 activations");
    require(precision == kWxA16, "q4/q5/q6 A8 plans are not admitted on gfx950");
    if (implementation == kFusedResearch) {
        require(bits == 4, "the fused research path exists for q4 only on gfx950");
        plan.path = kDirect;
    } else {
        plan.path = kChunkedDense;
    }
    plan.passes = 0;
    return plan;
}

void check_plan(const VRCPlan* plan) {
    require(plan, "null row-codec plan");
    const VRCPlan again = admit(plan->bits, plan->group, plan->precision, plan->dtype, plan->implementation);
    require(again.path == plan->path && again.passes == plan->passes, "row-codec plan does not come from prepare");
}

void pass(int status) {
    if (status != 0) throw std::runtime_error(venturi_blocks_error());
}

// Model::project for one matrix (qwen_runtime.cuh:365-390): out [tokens][n].
void project(const VRCPlan& plan, const void* x, const void* codes, const void* high, const void* scales, void* out,
             void* workspace, std::uint64_t available, int tokens, int n, int k, int padded, bool packed,
             hipStream_t stream) {
    if (plan.path == kQuantized) {
        if (!packed) pass(venturi_q8_dp4a_quantize(x, workspace, available, tokens, k, plan.passes, stream));
        pass(venturi_q8_dp4a_run(workspace, available, static_cast<const std::int8_t*>(codes), scales, out, tokens, n,
                                 k, padded, plan.passes, stream));
        return;
    }
    if (plan.bits == 8) {
        // Direct: the reference's head kernel (canonical bytes, as
        // row_codec_dispatch.cuh:30-38 runs it) up to 32 tokens; above that the
        // prefill GEMM on matrix cores where it applies (fp16, k % 8 == 0).
        const bool mfma = plan.dtype == kF16 && k % 8 == 0 && aligned(x, 16) && aligned(codes, 16);
        if (mfma && tokens > 32)
            pass(venturi_q8_prefill_run(x, static_cast<const std::int8_t*>(codes), scales, out, tokens, n, k, padded,
                                        plan.dtype, stream));
        else
            pass(venturi_q8_head_run(x, static_cast<const std::int8_t*>(codes), scales, out, tokens, n, k, padded,
                                     plan.dtype, stream));
        return;
    }
    if (plan.path == kDirect) {  // q4 fused research GEMV
        pass(venturi_q4_fused_run(x, codes, scales, out, tokens, n, k, padded, plan.dtype, stream));
        return;
    }
    // ChunkedDense: the W*A16 contract. From kDenseTokens tokens the reference's
    // own form (fp16 shadow chunks in the workspace + hipBLASLt) when the
    // geometry and the workspace allow it; else the fused matrix-core GEMM when
    // k % 8 == 0; else the reference-order expert GEMVs up to 64 tokens.
    if (tokens >= kDenseTokens && plan.dtype == kF16 && k % 8 == 0 && n % 8 == 0 && aligned(x, 16) &&
        aligned(out, 16) && workspace && aligned(workspace, 256) && available >= kDenseMinBytes + 32ull * k) {
        pass(venturi_row_dense_run(x, codes, high, scales, out, tokens, n, k, padded, plan.bits, plan.dtype, workspace,
                                   available, stream));
        return;
    }
    if (k % 8 == 0 && aligned(x, 16)) {
        pass(venturi_row_gemm_run(x, codes, high, scales, out, tokens, n, k, padded, plan.bits, plan.dtype, stream));
        return;
    }
    require(tokens <= 64 && plan.bits <= 5, "row-codec projection needs k % 8 == 0 here (or q4/q5 and <= 64 tokens)");
    const int status = plan.bits == 4
                           ? venturi_q4_linear(x, codes, scales, out, tokens, n, k, padded, stream)
                           : venturi_q5_linear(x, codes, high, scales, out, tokens, n, k, padded, stream);
    require(status == 0, "row-codec GEMV launch failed");
}

}  // namespace
}  // namespace vt

#define VT_EXPORT extern "C" __attribute__((visibility("default")))

VT_EXPORT int venturi_rowcodec_prepare(int bits, int group, int precision, int dtype, int implementation,
                                       VRCPlan* plan) {
    const bool ok = vt::host_guarded([&] {
        vt::require(plan, "null row-codec plan");
        *plan = vt::admit(bits, group, precision, dtype, implementation);
    });
    return ok ? 0 : -1;
}

VT_EXPORT uint64_t venturi_rowcodec_workspace_bytes(const VRCPlan* plan, int tokens, int k) {
    std::uint64_t bytes = 0;
    vt::host_guarded([&] {
        vt::check_plan(plan);
        if (plan->path == vt::kQuantized) {
            bytes = venturi_q8_dp4a_bytes(tokens, k, plan->passes);
            vt::require(bytes > 0, "invalid A8 geometry");
        } else if (plan->path == vt::kChunkedDense && plan->dtype == vt::kF16 && tokens >= vt::kDenseTokens) {
            vt::require(k > 0, "invalid row-codec geometry");
            bytes = vt::kDenseBytes;
        }
    });
    return bytes;
}

VT_EXPORT int venturi_rowcodec_project(const VRCPlan* plan, const void* x, const void* codes, const void* high,
                                       const void* scales, void* out, void* workspace, uint64_t available, int tokens,
                                       int n, int k, int padded, int packed, void* stream) {
    return vt::guarded([&] {
        vt::check_plan(plan);
        vt::require(packed == 0 || (packed == 1 && plan->path == vt::kQuantized),
                    "packed reuse applies to A8 plans only");
        vt::project(*plan, x, codes, high, scales, out, workspace, available, tokens, n, k, padded, packed != 0,
                    static_cast<hipStream_t>(stream));
    });
}
