/*
 * libbootstrap_hip.so — C ABI of the MI355X (gfx950) INT8 KV-cache path.
 *
 * It replaces native/bridge.mm (the Objective-C++ Metal bridge) for the INT8
 * full-attention KV path: the engine keeps its KV allocator, grow policy and
 * checkpoint logic and keeps binding these symbols by P/Invoke
 * (src/Bootstrap.Engine/Metal.cs:26-41); only the library name changes from
 * "bootstrap_metal" to "bootstrap_hip" (Metal.cs:18-24).
 *
 * Plain pointers and sizes only. Every pointer named `ctx` is a context from
 * boot_create, every `buf` a buffer from boot_buffer/boot_map.
 *
 * Errors: handle-returning functions return NULL, operations return 0; the
 * message is then read with boot_error(ctx) (bridge.mm:69, Metal.cs:69).
 * Threading: a context is not thread-safe; one thread drives it, as the engine's
 * single inference semaphore does (Api.cs:15,26). Buffers are device HBM: the
 * host reads/writes them only through boot_read/boot_write/boot_copy.
 */
#ifndef BOOTSTRAP_HIP_H
#define BOOTSTRAP_HIP_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* 64-byte kernel argument block bound at Metal buffer index 15.
 * Metal.cs:6-12 (KernelArgs), kernels.metal:6 (struct P). */
typedef struct boot_kernel_args {
    uint32_t n, m, k, kind, pos, flags, a, b;
    float eps, theta, scale, value;
    uint32_t c, d, e, f;
} boot_kernel_args;

/* bridge.mm:58-68. Creates the device context (HIP device 0, one stream of
 * default priority). `source` is accepted for signature compatibility and
 * ignored: the gfx950 kernels are compiled into this library. NULL if no
 * usable gfx950 device exists. */
void *boot_create(const char *source);
/* bridge.mm:69. Last error message of the context (never NULL). */
const char *boot_error(void *ctx);
/* bridge.mm:112-116. Waits for outstanding work, frees every buffer the
 * context still owns and the context itself. */
void boot_destroy(void *ctx);
/* bridge.mm:117-122. Zero-filled device allocation of `bytes` bytes. */
void *boot_buffer(void *ctx, uint64_t bytes);
/* bridge.mm:123-134. Reads a file into a new device buffer (no mmap of HBM). */
void *boot_map(void *ctx, const char *path);
/* bridge.mm:135. Device buffers have no host mapping: always NULL. Callers use
 * boot_read/boot_write instead of spans (Metal.cs:49-53). */
void *boot_contents(void *buf);
/* bridge.mm:136. */
void boot_release_buffer(void *buf);
/* bridge.mm:137. Bytes currently allocated through this context. */
uint64_t boot_allocated(void *ctx);
/* bridge.mm:138-144. Opens a command; fails if one is already active. */
int boot_begin(void *ctx);
/* bridge.mm:145-150. Enqueues a zero fill of the whole buffer (a fill kernel,
 * no memset node). Requires an active command. */
int boot_clear(void *ctx, void *buf);
/* bridge.mm:151-206. Enqueues kernel `name` with `count` buffer bindings
 * (buffers[i] + offsets[i] bound at index i) and the 64-byte argument block.
 * Launch geometry is chosen by the library from the arguments; x..tz are the
 * caller's Metal thread counts and are only validated for consistency where
 * a kernel needs them. `indirect` must be NULL (no INT8 kernel is indirect).
 * Sizes are validated against the bound buffers before launch. A dispatch with
 * no rows (M = 0; attention_softmax: no 256-thread row groups) launches nothing
 * and succeeds, as a zero-thread Metal dispatch does, except the single-row
 * attention_decode_append_int8, which requires M = 1. */
int boot_dispatch(void *ctx, const char *name, void **buffers, const uint64_t *offsets, int count,
                  const void *params, int param_bytes, uint32_t x, uint32_t y, uint32_t z,
                  uint32_t tx, uint32_t ty, uint32_t tz, void *indirect, uint64_t indirect_offset);
/* bridge.mm:207-280. Closes the command and blocks until the GPU finished it;
 * 0 (with the HIP error text) if any enqueued work failed. */
int boot_end(void *ctx);

/* bridge.mm:70. Serialized per-dispatch timing (BOOTSTRAP_PROFILE equivalent). */
void boot_profile(void *ctx, int enabled);
/* bridge.mm:71-94. Resets wall accounting; sample_attention 1 samples the
 * attention kernels, 2 every kernel, with HIP events on the context stream,
 * keyed by dispatch name; 3 times each kernel of the path alone, keyed by kernel
 * function, with events stamped by its own dispatch (no marker packets). */
int boot_wall_reset(void *ctx, int sample_attention);
/* bridge.mm:95-105. wall[7] = {gpu s, encode s, commit s, wait s, commands,
 * dispatches, resolve s}; attention[6] = {qk s, softmax s, av s, counts x3}. */
void boot_wall_read(void *ctx, double *wall, double *attention);
/* bridge.mm:106-111. JSON array [{"kernel","gpu_ms","count"}] of sampled
 * per-kernel GPU time since boot_wall_reset. */
const char *boot_kernel_wall_json(void *ctx);

/* ---- Additions required because HBM is not host-addressable (the engine's
 * span copies at QwenEngine.cs:80 and buffer fills become these calls). ---- */

/* Size in bytes of a buffer. */
uint64_t boot_buffer_size(void *buf);
/* Device-to-device copy (the Grow copy, QwenEngine.cs:76-82). Enqueued in the
 * active command, or synchronous when no command is active. */
int boot_copy(void *ctx, void *dst, uint64_t dst_offset, void *src, uint64_t src_offset, uint64_t bytes);
/* Host -> device and device -> host copies; only outside a command
 * (the engine touches buffers only between End and Begin, QwenEngine.cs:89). */
int boot_write(void *ctx, void *buf, uint64_t offset, const void *host, uint64_t bytes);
int boot_read(void *ctx, void *buf, uint64_t offset, void *host, uint64_t bytes);

/* ---- No counterpart in the reference. For callers that cannot allocate device memory
 * (tight serving loops, harnesses that forbid hipMalloc). ----
 *
 * boot_dispatch with the same arguments and outputs, except that kernels whose launch needs
 * scratch (split-K partials of attention_decode_int8, attention_decode_append_int8, the
 * attention_online_* prefill names and batch_attention_values_int8; the chunk statistics of
 * attention_softmax) draw it from a static 72 MiB device array of the library instead of the
 * context workspace; it calls no hipMalloc/hipFree or other allocating routine and records no
 * timing sample. Requests larger than 72 MiB are rejected (0, with the size in boot_error) before
 * any launch; 72 MiB covers prefill chunks of up to 512 rows and of 2048 rows on 256 CUs,
 * single-token decode up to the 262144 window, and the scalar reader for 8 rows up to 262144
 * keys (values partials: rows x 2 x keys / 512 x 8 KiB, 64 MiB there). One GPU has one array: the first split-K call of a command claims it
 * for that context until the command's boot_end, and a split-K call of another context meanwhile
 * fails (0, "held by another context's command") instead of racing; calls in one context's
 * command are ordered on its stream. The context's stream is the library's own and boot_end
 * synchronizes it, so this entry point does not make the library's work capturable into a HIP
 * graph. */
int boot_dispatch_noalloc(void *ctx, const char *name, void **buffers, const uint64_t *offsets, int count,
                          const void *params, int param_bytes, uint32_t x, uint32_t y, uint32_t z,
                          uint32_t tx, uint32_t ty, uint32_t tz, void *indirect, uint64_t indirect_offset);

#ifdef __cplusplus
}
#endif
#endif
