// Library identity and the per-thread error channel shared by every export.
#include <hip/hip_runtime.h>

#include <string>

namespace vt {
namespace {
thread_local std::string error_text;
}
void set_error(const char* text) { error_text = text; }
void clear_error() { error_text.clear(); }
}  // namespace vt

#define VT_EXPORT extern "C" __attribute__((visibility("default")))

// Reference: blocks.cu:650-652. The ABI number is the reference's (18) for the
// shared signatures; the architecture tag names this build's target.
VT_EXPORT int venturi_blocks_abi() { return 18; }
VT_EXPORT int venturi_blocks_arch() { return 950; }
VT_EXPORT const char* venturi_blocks_error() { return vt::error_text.c_str(); }
