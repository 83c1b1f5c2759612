// Shared host/device declarations of libbootstrap_hip.so (gfx950 only).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/bootstrap_hip.h"

namespace boot {

// Model geometry the INT8 path is specialised to (kernels.metal:142-146,
// QwenEngine.cs:61): 16 query heads, 2 KV heads, head dim 256, GQA 8:1.
constexpr int kQHeads = 16;
constexpr int kKvHeads = 2;
constexpr int kHeadDim = 256;
constexpr int kGroup = 8;
constexpr int kPageTokens = 256;          // V page: 256 tokens x 256 dims per KV head
constexpr uint64_t kPageBytes = 65536;    // one (page, head) block of V codes

// One buffer binding as the kernel sees it: base + offset and the bytes that
// remain in the buffer after the offset.
struct View {
    char *ptr;
    uint64_t bytes;
};

struct Context;

// A launcher validates its bindings against the argument block and enqueues
// its kernels on the context stream. Returns nullptr or an error message.
using Launcher = const char *(*)(Context &, const View *, int, const boot_kernel_args &,
                                 const uint32_t grid[6]);

// Stream, per-context scratch memory and error state, owned by the shim.
hipStream_t context_stream(Context &c);
// Device scratch of at least `bytes` bytes that stays valid until the next
// call; grows (with a stream sync) only when the request exceeds what is held.
void *context_workspace(Context &c, uint64_t bytes);
// CU count of the device, for split decisions.
int context_cus(Context &c);
// Ends the current timing sample of a multi-kernel dispatch and starts one
// named `name` (no-op unless kernel sampling is on).
void context_split(Context &c, const char *name);
// Kernel-exact timing: in that wall-timing mode, returns start/stop events for
// hipExtLaunchKernelGGL, which stamps them from the dispatch packet itself (no
// marker packets on the stream), and records them as a sample named `kernel`;
// otherwise returns null events.
void context_kernel_events(Context &c, const char *kernel, hipEvent_t *start, hipEvent_t *stop);

// Enqueues `f` on the context stream, through hipExtLaunchKernelGGL with
// kernel-exact events when that mode is on (a slower host path), else as a plain
// launch. The arguments are converted to the kernel's parameter types first: the
// extended launch packs them by the types it is given.
template <typename... Params, typename... Args>
inline void launch_timed(Context &c, const char *kernel, void (*f)(Params...), dim3 grid, dim3 block, Args... args) {
    hipEvent_t start = nullptr, stop = nullptr;
    context_kernel_events(c, kernel, &start, &stop);
    if (start)
        hipExtLaunchKernelGGL(f, grid, block, 0, context_stream(c), start, stop, 0, static_cast<Params>(args)...);
    else
        f<<<grid, block, 0, context_stream(c)>>>(static_cast<Params>(args)...);
}

// Byte offset of the V code for (vector = token*2 + head, dimension d).
// kernels.metal:126-128 (int8_value_index).
__host__ __device__ inline uint64_t value_index(uint64_t vector, uint32_t d) {
    uint64_t token = vector >> 1, head = vector & 1;
    return ((token >> 8) * 2 + head) * kPageBytes + (uint64_t)d * 256 + (token & 255);
}

// Smallest V buffer that holds tokens [0, length): whole pages.
__host__ __device__ inline uint64_t value_bytes(uint64_t length) {
    return (length + 255) / 256 * 256 * 512;
}

// Registered launchers (one per reference kernel name the path services).
const char *launch_kv_store_int8(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_batch_rope_int8(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_query_grouped_half(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_prepare_fused_int8(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_rmsnorm(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_batch_split_q(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_online_int8(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_online_fp16(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_batch_rope_half(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_prepare_fused_half(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_decode_int8(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
// attention_online_int8 for chunks of at most 64 rows over a short history, through the decode
// kernel (bindings validated by the prefill launcher)
const char *launch_online_int8_as_decode(Context &, const View *, const boot_kernel_args &);
const char *launch_decode_append_int8(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_scores_int8(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_softmax(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);
const char *launch_values_int8(Context &, const View *, int, const boot_kernel_args &, const uint32_t *);

// Zero fill used by boot_clear and boot_buffer (no memset node is recorded).
hipError_t fill_zero(void *ptr, uint64_t bytes, hipStream_t stream);

}  // namespace boot

// Validation helper for launchers.
#define BOOT_REQUIRE(cond, msg) \
    do {                        \
        if (!(cond)) return msg; \
    } while (0)
