// Exports of the reference's operator ABI that lie outside the quantized-linear
// path (sampling, attention, RoPE, gated delta-net, the fp32 and fp16 dense
// embedding / linear helpers). The reference's Python backend binds every one
// of them when it is constructed (blocks.py:336-427), so a binding written for
// the reference must find them here to load this library at all. Each keeps the
// reference's C signature (ops_api.h) and fails like any rejected call: -1 with
// a per-thread message, no HIP call, no output written.
#include <cstddef>
#include <cstdint>

namespace vt {
void set_error(const char* text);
}

#define VT_EXPORT extern "C" __attribute__((visibility("default")))

namespace {
int absent(const char* message) {
    vt::set_error(message);
    return -1;
}
}  // namespace

// ops_api.h:46-47
VT_EXPORT int venturi_greedy_run(const void*, std::int64_t*, void*, std::size_t, int, int, int, void*) {
    return absent("venturi_greedy_run: not built for gfx950 (outside the quantized-linear path)");
}

// ops_api.h:30-31
VT_EXPORT int venturi_fp32_linear_run(const void*, const float*, void*, int, int, int, int, void*) {
    return absent("venturi_fp32_linear_run: not built for gfx950 (outside the quantized-linear path)");
}

// ops_api.h:95-96
VT_EXPORT int venturi_rope_run(const void*, const float*, const float*, void*, int, int, int, int, int, int, void*) {
    return absent("venturi_rope_run: not built for gfx950 (outside the quantized-linear path)");
}

// ops_api.h:87-90
VT_EXPORT int venturi_qwen_qk_run(const void*, const void*, const float*, const float*, const float*, const float*,
                                  void*, void*, int, int, int, int, int, int, float, void*) {
    return absent("venturi_qwen_qk_run: not built for gfx950 (outside the quantized-linear path)");
}

// ops_api.h:85-86
VT_EXPORT int venturi_qwen_gate_run(const void*, const void*, void*, int, int, int, int, void*) {
    return absent("venturi_qwen_gate_run: not built for gfx950 (outside the quantized-linear path)");
}

// ops_api.h:13-15
VT_EXPORT int venturi_attention_run(const void*, const void*, const void*, void*, int, int, int, int, int, int, float,
                                    void*) {
    return absent("venturi_attention_run: not built for gfx950 (outside the quantized-linear path)");
}

// ops_api.h:28-29
VT_EXPORT int venturi_embedding_run(const void*, const std::int64_t*, void*, int, int, int, int, void*) {
    return absent("venturi_embedding_run: not built for gfx950 (outside the quantized-linear path)");
}

// ops_api.h:42-44
VT_EXPORT int venturi_gdn_run(const void*, const void*, const void*, const float*, const float*, const float*, void*,
                              float*, int, int, int, int, int, int, int, int, float, void*) {
    return absent("venturi_gdn_run: not built for gfx950 (outside the quantized-linear path)");
}

// ops_api.h:19-20
VT_EXPORT int venturi_conv_run(const void*, const void*, const void*, void*, void*, int, int, int, int, int, void*) {
    return absent("venturi_conv_run: not built for gfx950 (outside the quantized-linear path)");
}

// ops_api.h:34-35
VT_EXPORT int venturi_gates_run(const void*, const void*, const float*, const float*, float*, float*, int, int, int, int,
                                void*) {
    return absent("venturi_gates_run: not built for gfx950 (outside the quantized-linear path)");
}

// ops_api.h:32-33
VT_EXPORT int venturi_gated_rms_run(const void*, const void*, const void*, void*, int, int, int, int, int, float,
                                    void*) {
    return absent("venturi_gated_rms_run: not built for gfx950 (outside the quantized-linear path)");
}
