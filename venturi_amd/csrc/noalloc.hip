// The tiled Q8 projection for callers that cannot allocate (code under HIP
// graph capture, serving loops, harnesses that forbid hipMalloc).
//
// venturi_q8_tiled_run takes the exchange slots of launches that split K over
// two workgroups from a caller-owned workspace. This variant keeps them in a
// file-scope device array instead: 1 MiB, enough for every split shape (a
// launch splits only while its grid fits one workgroup per CU, i.e. at most
// 512 row blocks x 32 tokens x 64 bytes). Each GPU the library runs on holds
// its own copy until the process ends. The slots must start idle (the
// signalling-NaN pattern of the tiled kernels, not zero): the first call on a
// device fills them with a kernel on the caller's stream, outside graph
// capture, and waits for that fill (so later calls on any stream find idle
// slots); every projection leaves them idle again. All calls on one GPU share
// the array, so calls that overlap in time on one GPU race, and a race can
// leave slots non-idle for every later call on that GPU: nothing re-arms the
// array, so recovery from an overlapping call is a new process.
#include "common.hpp"

#include <mutex>

namespace vt {

std::size_t q8_tiled_workspace_bytes(int tokens, int n, bool swiglu);
void q8_tiled_workspace_init(void* workspace, std::size_t bytes, hipStream_t stream);
void q8_tiled_launch(const void* x, const void* codes, const void* scales, void* out, int tokens, int n, int k,
                     int padded, int dtype, bool swiglu, void* workspace, std::size_t workspace_bytes,
                     hipStream_t stream);

namespace {

constexpr std::size_t kScratchBytes = std::size_t{1} << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned long long scratch[kScratchBytes / sizeof(unsigned long long)];

std::mutex scratch_lock;
void* scratch_address[kMaxDevices] = {};

// The current device's copy of `scratch`, idle. The first call on a device
// resolves the array's device address (the host-side name is no device
// address) and fills it on `stream`.
void* device_scratch(hipStream_t stream) {
    int device = -1;
    check(hipGetDevice(&device));
    require(device >= 0 && device < kMaxDevices, "device ordinal outside the static scratch table");
    std::lock_guard<std::mutex> lock(scratch_lock);
    if (!scratch_address[device]) {
        hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
        check(hipStreamIsCapturing(stream, &status));
        require(status == hipStreamCaptureStatusNone,
                "the first venturi_q8_tiled_run_noalloc call on a device must run outside graph capture "
                "(it initialises the static exchange slots)");
        void* address = nullptr;
        check(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)));
        q8_tiled_workspace_init(address, kScratchBytes, stream);
        check(hipGetLastError());
        // Finish the fill before any call on another stream can reach the slots:
        // the split-K exchange reads every non-idle word as a partner's partial.
        check(hipStreamSynchronize(stream));
        scratch_address[device] = address;
    }
    return scratch_address[device];
}

}  // namespace
}  // namespace vt

// No counterpart in the reference: venturi_q8_tiled_run without the workspace
// arguments, for callers that cannot allocate.
extern "C" __attribute__((visibility("default"))) int venturi_q8_tiled_run_noalloc(const void* x, const void* codes,
                                                                                  const void* scales, void* out,
                                                                                  int tokens, int n, int k,
                                                                                  int padded, int dtype,
                                                                                  void* stream) {
    return vt::guarded([&] {
        const auto s = static_cast<hipStream_t>(stream);
        const std::size_t need = vt::q8_tiled_workspace_bytes(tokens, n, false);
        vt::require(need <= vt::kScratchBytes, "the projection's exchange slots exceed the 1 MiB static scratch");
        void* slots = need ? vt::device_scratch(s) : nullptr;
        vt::q8_tiled_launch(x, codes, scales, out, tokens, n, k, padded, dtype, false, slots, need, s);
    });
}
