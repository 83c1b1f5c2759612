// libbootstrap_hip.so host side: the boot_* C ABI that replaces the Metal
// bridge (native/bridge.mm:57-281) for the INT8 KV-cache path.
//
// One context = one HIP device (device 0, must be gfx950) and one stream of
// default priority. A command (boot_begin .. boot_end) enqueues dispatches on
// that stream; boot_end blocks until they finished (bridge.mm:214-217).
// Dispatch is by kernel name (bridge.mm:153-160): each name maps to a launcher
// that validates the bound buffer sizes against the argument block and picks
// its own gfx950 launch geometry.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "common.h"

namespace boot {

// Split-K scratch of boot_dispatch_noalloc (the attention kernels' per-split partials): 72 MiB,
// enough for prefill chunks of up to 512 rows and of 2048 rows on 256 CUs (at most 279 partials
// of 265,216 bytes) and for single-token decode up to the 262144 window (about 2 MiB). Each
// device holds its own copy until the process ends; the host reaches it only through the
// address kept per device below.
constexpr uint64_t kStaticScratchBytes = 72ull << 20;

}  // namespace boot

static __device__ __align__(256) unsigned char scratch[boot::kStaticScratchBytes];

namespace boot {

namespace {
constexpr int kMaxDevices = 64;
std::once_flag scratch_once[kMaxDevices];
void *scratch_address[kMaxDevices];
hipError_t scratch_status[kMaxDevices];
// The context whose open command holds the device's scratch (from its first split-K
// boot_dispatch_noalloc until its boot_end), or null: a noalloc split-K dispatch of any other
// context meanwhile is refused instead of racing on the partials.
std::atomic<const void *> scratch_owner[kMaxDevices];

// Device address of `scratch` on the current device, looked up once per device (the array's
// name is a host-side stand-in, never a device address). Null with the HIP error if the lookup
// failed.
void *static_scratch(int device, hipError_t *status) {
    if (device < 0 || device >= kMaxDevices) {
        *status = hipErrorInvalidDevice;
        return nullptr;
    }
    std::call_once(scratch_once[device], [device] {
        void *ptr = nullptr;
        scratch_status[device] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        scratch_address[device] = scratch_status[device] == hipSuccess ? ptr : nullptr;
    });
    *status = scratch_status[device];
    return scratch_address[device];
}
}  // namespace

struct Buffer {
    Context *ctx;
    void *ptr;
    uint64_t bytes;
};

struct Sample {
    std::string name;
    hipEvent_t start, end;
    int kind;
};

struct Context {
    int device = 0;
    int cus = 0;
    hipStream_t stream = nullptr;
    std::string error;
    bool active = false;
    std::unordered_set<Buffer *> buffers;
    uint64_t allocated = 0;
    void *workspace = nullptr;
    uint64_t workspace_bytes = 0;
    // boot_dispatch_noalloc: the device's static scratch replaces the workspace and no
    // timing event is recorded while `noalloc` is set
    bool noalloc = false;
    void *scratch = nullptr;
    hipError_t scratch_status = hipSuccess;
    uint64_t scratch_request = 0;   // bytes the last refused request asked for
    bool scratch_busy = false;      // the last request found the scratch held by another context
    std::string workspace_error;    // the HIP error of the last failed workspace growth
    // serialized per-dispatch profiling (bridge.mm:61,198-204)
    bool profile = false;
    std::map<std::string, std::pair<double, uint64_t>> timings;
    // wall accounting and sampled kernel timing (bridge.mm:71-111)
    bool wall_enabled = false;
    int sample_mode = 0;
    double wall[7] = {};
    double attention[6] = {};
    std::map<std::string, std::pair<double, uint64_t>> kernel_wall;
    std::string kernel_json;
    std::vector<hipEvent_t> events;
    size_t events_used = 0;
    std::vector<Sample> samples;
    hipEvent_t command_start = nullptr, command_end = nullptr;
    double begin_time = 0;
    // sample being recorded for the current dispatch (see context_split)
    bool sampling = false;
    std::string current_name;
    hipEvent_t current_start = nullptr;
    int current_kind = -1;
};

namespace {

double wall_now() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

bool fail(Context *c, const std::string &message) {
    c->error = message;
    return false;
}

bool hip_ok(Context *c, hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    c->error = std::string(what) + ": " + hipGetErrorString(e);
    return false;
}

hipEvent_t next_event(Context *c) {
    if (c->events_used == c->events.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        c->events.push_back(e);
    }
    return c->events[c->events_used++];
}

// An event recorded on the context stream, or null when that fails (the sample it
// belonged to is then dropped; timing never fails a command).
hipEvent_t record(Context *c) {
    hipEvent_t e = next_event(c);
    if (e && hipEventRecord(e, c->stream) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return e;
}

struct Entry {
    Launcher launch;
    int kind;  // attention sample kind: 0 QK, 1 softmax, 2 AV, 3 fused online/decode, -1 other
};

const std::unordered_map<std::string, Entry> &registry() {
    static const std::unordered_map<std::string, Entry> table = {
        {"kv_store_int8", {launch_kv_store_int8, -1}},
        {"batch_rope_int8", {launch_batch_rope_int8, -1}},
        {"attention_query_grouped_half", {launch_query_grouped_half, -1}},
        {"attention_prepare_fused_int8", {launch_prepare_fused_int8, -1}},
        {"rmsnorm", {launch_rmsnorm, -1}},
        {"batch_split_q", {launch_batch_split_q, -1}},
        {"attention_online_int8_q32_k256_r2", {launch_online_int8, 3}},
        {"attention_online_int8", {launch_online_int8, 3}},
        {"attention_online_int8_q32_k128", {launch_online_int8, 3}},
        {"attention_decode_int8", {launch_decode_int8, 3}},
        {"attention_decode_append_int8", {launch_decode_append_int8, 3}},
        {"attention_online_q32_k256_s8_g8_r2", {launch_online_fp16, 3}},
        {"batch_rope", {launch_batch_rope_half, -1}},
        {"attention_prepare_fused", {launch_prepare_fused_half, -1}},
        {"batch_attention_scores_int8", {launch_scores_int8, 0}},
        {"attention_softmax", {launch_softmax, 1}},
        {"batch_attention_values_int8", {launch_values_int8, 2}},
    };
    return table;
}

Buffer *as_buffer(Context *c, void *handle) {
    Buffer *b = static_cast<Buffer *>(handle);
    if (!b || c->buffers.find(b) == c->buffers.end()) return nullptr;
    return b;
}

}  // namespace

hipStream_t context_stream(Context &c) { return c.stream; }
int context_cus(Context &c) { return c.cus; }

void *context_workspace(Context &c, uint64_t bytes) {
    if (c.noalloc) {
        if (!c.scratch || bytes > kStaticScratchBytes) {
            c.scratch_request = bytes;
            return nullptr;
        }
        const void *expected = nullptr;
        if (!scratch_owner[c.device].compare_exchange_strong(expected, &c) && expected != &c) {
            c.scratch_busy = true;
            return nullptr;
        }
        return c.scratch;
    }
    if (bytes <= c.workspace_bytes) return c.workspace;
    // A failed call's error is read back here, so that the launch check of a later dispatch
    // (hipGetLastError) does not report it again, and kept for this dispatch's message.
    auto failed = [&c](hipError_t e, const char *what) -> void * {
        (void)hipGetLastError();
        c.workspace_error = std::string(what) + ": " + hipGetErrorString(e);
        return nullptr;
    };
    // Grow: the old scratch may still be read by enqueued work.
    hipError_t e = hipStreamSynchronize(c.stream);
    if (e != hipSuccess) return failed(e, "stream synchronize before the workspace grows");
    if (c.workspace) {
        e = hipFree(c.workspace);
        if (e != hipSuccess) return failed(e, "hipFree of the old workspace");
        c.allocated -= c.workspace_bytes;
    }
    c.workspace = nullptr;
    c.workspace_bytes = 0;
    uint64_t want = bytes < (64ull << 20) ? (64ull << 20) : bytes;
    e = hipMalloc(&c.workspace, want);
    if (e != hipSuccess) {
        c.workspace = nullptr;
        return failed(e, ("hipMalloc of " + std::to_string(want) + " bytes").c_str());
    }
    c.workspace_bytes = want;
    c.allocated += want;
    return c.workspace;
}

void context_kernel_events(Context &c, const char *kernel, hipEvent_t *start, hipEvent_t *stop) {
    *start = *stop = nullptr;
    if (c.noalloc || !c.wall_enabled || c.sample_mode != 3 || !c.active) return;
    hipEvent_t a = next_event(&c), b = next_event(&c);
    if (!a || !b) return;
    *start = a;
    *stop = b;
    c.samples.push_back({kernel, a, b, -1});
}

// Ends the current sample of a multi-kernel dispatch and starts one named
// `name` (used to time a split-K combine apart from its main kernel).
void context_split(Context &c, const char *name) {
    if (c.noalloc || !c.sampling) return;
    hipEvent_t e = record(&c);
    c.samples.push_back({c.current_name, c.current_start, e, c.current_kind});
    c.current_name = name;
    c.current_start = e;
    c.current_kind = -1;
}

// Gives the device's scratch back if this context's command held it; called once the context's
// stream has drained (its kernels no longer read or write the scratch).
void release_scratch(Context &c) {
    const void *self = &c;
    scratch_owner[c.device].compare_exchange_strong(self, nullptr);
}

}  // namespace boot

using namespace boot;

extern "C" {

void *boot_create(const char *source) {
    (void)source;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count < 1) {
        fprintf(stderr, "bootstrap_hip: no HIP device\n");
        return nullptr;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return nullptr;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        fprintf(stderr, "bootstrap_hip: device 0 is %s; this library is built for gfx950 only\n", prop.gcnArchName);
        return nullptr;
    }
    if (hipSetDevice(0) != hipSuccess) return nullptr;
    Context *c = new Context();
    c->cus = prop.multiProcessorCount;
    // the static scratch of boot_dispatch_noalloc, once per device with it current; a failed
    // lookup fails only that entry point (with this error)
    c->scratch = static_scratch(0, &c->scratch_status);
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return nullptr;
    }
    c->profile = getenv("BOOTSTRAP_PROFILE") != nullptr;
    return c;
}

const char *boot_error(void *handle) { return static_cast<Context *>(handle)->error.c_str(); }

void boot_profile(void *handle, int enabled) {
    Context *c = static_cast<Context *>(handle);
    c->profile = enabled != 0;
    c->timings.clear();
}

int boot_wall_reset(void *handle, int sample_attention) {
    Context *c = static_cast<Context *>(handle);
    if (c->active || c->profile) return fail(c, "Wall profiling requires no active command and serial profiling disabled");
    c->wall_enabled = true;
    c->sample_mode = sample_attention;
    c->kernel_wall.clear();
    std::fill_n(c->wall, 7, 0.0);
    std::fill_n(c->attention, 6, 0.0);
    return 1;
}

void boot_wall_read(void *handle, double *wall, double *attention) {
    Context *c = static_cast<Context *>(handle);
    std::copy_n(c->wall, 7, wall);
    std::copy_n(c->attention, 6, attention);
}

const char *boot_kernel_wall_json(void *handle) {
    Context *c = static_cast<Context *>(handle);
    std::string s = "[";
    bool first = true;
    for (auto &item : c->kernel_wall) {
        char buf[512];
        snprintf(buf, sizeof buf, "%s{\"kernel\":\"%s\",\"gpu_ms\":%.9g,\"count\":%llu}", first ? "" : ",",
                 item.first.c_str(), item.second.first * 1000.0, (unsigned long long)item.second.second);
        s += buf;
        first = false;
    }
    s += "]";
    c->kernel_json = s;
    return c->kernel_json.c_str();
}

void boot_destroy(void *handle) {
    Context *c = static_cast<Context *>(handle);
    if (!c) return;
    // teardown: an error here has no caller left to reach, so each call is best effort
    (void)hipStreamSynchronize(c->stream);
    release_scratch(*c);
    if (c->profile)
        for (auto &entry : c->timings)
            fprintf(stderr, "GPU_DIAGNOSTIC %s count=%llu gpu_ms=%.6f\n", entry.first.c_str(),
                    (unsigned long long)entry.second.second, entry.second.first * 1000);
    for (Buffer *b : c->buffers) {
        (void)hipFree(b->ptr);
        delete b;
    }
    if (c->workspace) (void)hipFree(c->workspace);
    for (hipEvent_t e : c->events) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(c->stream);
    delete c;
}

void *boot_buffer(void *handle, uint64_t bytes) {
    Context *c = static_cast<Context *>(handle);
    if (bytes == 0) bytes = 4;
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();   // clear the error so the next call does not report it
        c->error = "HIP buffer allocation failed";
        return nullptr;
    }
    if (fill_zero(p, bytes, c->stream) != hipSuccess || hipStreamSynchronize(c->stream) != hipSuccess) {
        (void)hipFree(p);   // the fill error is the one reported
        c->error = "HIP buffer zero fill failed";
        return nullptr;
    }
    Buffer *b = new Buffer{c, p, bytes};
    c->buffers.insert(b);
    c->allocated += bytes;
    return b;
}

void *boot_map(void *handle, const char *path) {
    Context *c = static_cast<Context *>(handle);
    FILE *f = fopen(path, "rb");
    if (!f) {
        c->error = "Cannot open weight file";
        return nullptr;
    }
    fseek(f, 0, SEEK_END);
    long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (size < 0) {
        fclose(f);
        c->error = "Cannot stat weight file";
        return nullptr;
    }
    Buffer *b = static_cast<Buffer *>(boot_buffer(c, (uint64_t)size));
    if (!b) {
        fclose(f);
        return nullptr;
    }
    std::vector<char> chunk(1 << 24);
    uint64_t done = 0;
    while (done < (uint64_t)size) {
        size_t n = fread(chunk.data(), 1, chunk.size(), f);
        if (n == 0) break;
        if (hipMemcpy((char *)b->ptr + done, chunk.data(), n, hipMemcpyHostToDevice) != hipSuccess) break;
        done += n;
    }
    fclose(f);
    if (done != (uint64_t)size) {
        boot_release_buffer(b);
        c->error = "Weight file read failed";
        return nullptr;
    }
    return b;
}

void *boot_contents(void *handle) {
    (void)handle;
    return nullptr;  // HBM is not host-addressable; use boot_read/boot_write
}

uint64_t boot_buffer_size(void *handle) { return handle ? static_cast<Buffer *>(handle)->bytes : 0; }

void boot_release_buffer(void *handle) {
    Buffer *b = static_cast<Buffer *>(handle);
    if (!b) return;
    Context *c = b->ctx;
    // enqueued work may still read it; the call returns nothing, so failures land in
    // the context's error text
    if (hipStreamSynchronize(c->stream) != hipSuccess) c->error = "boot_release_buffer: stream synchronize failed";
    if (hipFree(b->ptr) != hipSuccess) c->error = "boot_release_buffer: hipFree failed";
    c->allocated -= b->bytes;
    c->buffers.erase(b);
    delete b;
}

uint64_t boot_allocated(void *handle) { return static_cast<Context *>(handle)->allocated; }

int boot_begin(void *handle) {
    Context *c = static_cast<Context *>(handle);
    if (c->active) return fail(c, "An unfinished command is active");
    c->active = true;
    c->events_used = 0;
    c->samples.clear();
    if (c->wall_enabled) {
        c->begin_time = wall_now();
        c->command_start = record(c);
    }
    return 1;
}

int boot_clear(void *handle, void *buffer) {
    Context *c = static_cast<Context *>(handle);
    if (!c->active) return fail(c, "boot_clear requires an active command");
    Buffer *b = as_buffer(c, buffer);
    if (!b) return fail(c, "boot_clear: unknown buffer");
    return hip_ok(c, fill_zero(b->ptr, b->bytes, c->stream), "boot_clear");
}

}  // extern "C"

namespace {

// boot_dispatch and boot_dispatch_noalloc. With `noalloc` the kernel name is matched without
// building strings, no timing event is recorded and split-K launchers draw their partials from
// the device's static scratch, so the call allocates no device or host memory unless it fails.
int dispatch(Context *c, const char *name, void **buffers, const uint64_t *offsets, int count,
             const void *parameters, int parameter_bytes, uint32_t x, uint32_t y, uint32_t z,
             uint32_t tx, uint32_t ty, uint32_t tz, void *indirect, bool noalloc) {
    if (!c->active) return fail(c, "boot_dispatch requires an active command");
    const Entry *entry = nullptr;
    for (auto &item : registry())
        if (name && strcmp(item.first.c_str(), name) == 0) entry = &item.second;
    if (!entry) return fail(c, std::string("Unknown kernel: ") + (name ? name : "(null)"));
    if (indirect) return fail(c, std::string(name) + ": indirect dispatch is not supported by INT8 kernels");
    if (count < 0 || count > 31) return fail(c, std::string(name) + ": invalid binding count");
    if (!parameters || parameter_bytes < (int)sizeof(boot_kernel_args))
        return fail(c, std::string(name) + ": argument block must be 64 bytes");
    if (noalloc && !c->scratch)
        return fail(c, std::string("boot_dispatch_noalloc: static scratch unavailable: ") +
                           hipGetErrorString(c->scratch_status));
    View views[32];
    for (int i = 0; i < count; i++) {
        Buffer *b = as_buffer(c, buffers[i]);
        if (!b) return fail(c, std::string(name) + ": binding " + std::to_string(i) + " is not a buffer of this context");
        uint64_t off = offsets ? offsets[i] : 0;
        if (off > b->bytes) return fail(c, std::string(name) + ": binding " + std::to_string(i) + " offset beyond buffer");
        views[i] = {static_cast<char *>(b->ptr) + off, b->bytes - off};
    }
    boot_kernel_args p;
    memcpy(&p, parameters, sizeof p);
    const uint32_t grid[6] = {x, y, z, tx, ty, tz};
    const bool sample = !noalloc && c->wall_enabled &&
                        (c->sample_mode == 2 || (c->sample_mode == 1 && entry->kind >= 0));
    const bool serial = !noalloc && c->profile;
    hipEvent_t serial_start = nullptr;
    if (serial) serial_start = record(c);
    if (sample) {
        c->sampling = true;
        c->current_name = name;
        c->current_kind = entry->kind;
        c->current_start = record(c);
    }
    c->noalloc = noalloc;
    const char *message = entry->launch(*c, views, count, p, grid);
    c->noalloc = false;
    if (sample) {
        hipEvent_t e = record(c);
        c->samples.push_back({c->current_name, c->current_start, e, c->current_kind});
        c->sampling = false;
    }
    if (message && noalloc && c->scratch_busy) {
        c->scratch_busy = false;
        return fail(c, std::string(name) + ": the static scratch of boot_dispatch_noalloc is held by another "
                                           "context's command until its boot_end");
    }
    if (message && noalloc && c->scratch_request > kStaticScratchBytes) {
        const uint64_t asked = c->scratch_request;
        c->scratch_request = 0;
        return fail(c, std::string(name) + ": split partials need " + std::to_string(asked) +
                           " bytes, more than the " + std::to_string(kStaticScratchBytes) +
                           "-byte static scratch of boot_dispatch_noalloc");
    }
    if (message && !c->workspace_error.empty()) {
        const std::string detail = c->workspace_error;
        c->workspace_error.clear();
        return fail(c, std::string(name) + ": " + message + " (" + detail + ")");
    }
    if (message) return fail(c, std::string(name) + ": " + message);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(c, std::string(name) + ": launch failed: " + hipGetErrorString(e));
    if (c->wall_enabled) c->wall[5]++;
    if (serial) {
        hipEvent_t stop = record(c);
        if (!hip_ok(c, hipEventSynchronize(stop), name)) return 0;
        float ms = 0;
        if (hipEventElapsedTime(&ms, serial_start, stop) != hipSuccess) ms = 0;
        auto &t = c->timings[name];
        t.first += ms * 1e-3;
        t.second++;
        c->events_used = 0;
    }
    return 1;
}

}  // namespace

extern "C" {

int boot_dispatch(void *handle, const char *name, void **buffers, const uint64_t *offsets, int count,
                  const void *parameters, int parameter_bytes, uint32_t x, uint32_t y, uint32_t z,
                  uint32_t tx, uint32_t ty, uint32_t tz, void *indirect, uint64_t indirect_offset) {
    (void)indirect_offset;
    return dispatch(static_cast<Context *>(handle), name, buffers, offsets, count, parameters, parameter_bytes, x, y,
                    z, tx, ty, tz, indirect, false);
}

int boot_dispatch_noalloc(void *handle, const char *name, void **buffers, const uint64_t *offsets, int count,
                          const void *parameters, int parameter_bytes, uint32_t x, uint32_t y, uint32_t z,
                          uint32_t tx, uint32_t ty, uint32_t tz, void *indirect, uint64_t indirect_offset) {
    (void)indirect_offset;
    return dispatch(static_cast<Context *>(handle), name, buffers, offsets, count, parameters, parameter_bytes, x, y,
                    z, tx, ty, tz, indirect, true);
}

int boot_end(void *handle) {
    Context *c = static_cast<Context *>(handle);
    if (!c->active) return fail(c, "boot_end without an active command");
    double before = c->wall_enabled ? wall_now() : 0;
    if (c->wall_enabled) c->command_end = record(c);
    hipError_t e = hipStreamSynchronize(c->stream);
    c->active = false;
    if (e == hipSuccess) release_scratch(*c);
    if (e != hipSuccess) return hip_ok(c, e, "command failed");
    if (c->wall_enabled) {
        double done = wall_now();
        float ms = 0;
        if (c->command_start && c->command_end && hipEventElapsedTime(&ms, c->command_start, c->command_end) != hipSuccess)
            ms = 0;
        c->wall[0] += ms * 1e-3;
        c->wall[1] += before - c->begin_time;
        c->wall[3] += done - before;
        c->wall[4]++;
        for (auto &s : c->samples) {
            float sms = 0;
            if (!s.start || !s.end) continue;   // an event that failed to record: no sample
            if (hipEventElapsedTime(&sms, s.start, s.end) != hipSuccess) continue;
            auto &k = c->kernel_wall[s.name];
            k.first += sms * 1e-3;
            k.second++;
            if (s.kind >= 0 && s.kind < 3) {
                c->attention[s.kind] += sms * 1e-3;
                c->attention[3 + s.kind]++;
            }
        }
        c->wall[6] += wall_now() - done;
    }
    c->samples.clear();
    c->events_used = 0;
    return 1;
}

int boot_copy(void *handle, void *dst, uint64_t dst_offset, void *src, uint64_t src_offset, uint64_t bytes) {
    Context *c = static_cast<Context *>(handle);
    Buffer *d = as_buffer(c, dst), *s = as_buffer(c, src);
    if (!d || !s) return fail(c, "boot_copy: unknown buffer");
    if (dst_offset > d->bytes || bytes > d->bytes - dst_offset || src_offset > s->bytes || bytes > s->bytes - src_offset)
        return fail(c, "boot_copy: range exceeds buffer");
    if (bytes == 0) return 1;
    if (!hip_ok(c, hipMemcpyAsync((char *)d->ptr + dst_offset, (char *)s->ptr + src_offset, bytes,
                                  hipMemcpyDeviceToDevice, c->stream), "boot_copy"))
        return 0;
    if (!c->active) return hip_ok(c, hipStreamSynchronize(c->stream), "boot_copy");
    return 1;
}

int boot_write(void *handle, void *buffer, uint64_t offset, const void *host, uint64_t bytes) {
    Context *c = static_cast<Context *>(handle);
    if (c->active) return fail(c, "boot_write: the host touches buffers only between End and Begin");
    Buffer *b = as_buffer(c, buffer);
    if (!b) return fail(c, "boot_write: unknown buffer");
    if (offset > b->bytes || bytes > b->bytes - offset) return fail(c, "boot_write: range exceeds buffer");
    if (bytes == 0) return 1;
    if (!hip_ok(c, hipMemcpyAsync((char *)b->ptr + offset, host, bytes, hipMemcpyHostToDevice, c->stream), "boot_write"))
        return 0;
    return hip_ok(c, hipStreamSynchronize(c->stream), "boot_write");
}

int boot_read(void *handle, void *buffer, uint64_t offset, void *host, uint64_t bytes) {
    Context *c = static_cast<Context *>(handle);
    if (c->active) return fail(c, "boot_read: the host touches buffers only between End and Begin");
    Buffer *b = as_buffer(c, buffer);
    if (!b) return fail(c, "boot_read: unknown buffer");
    if (offset > b->bytes || bytes > b->bytes - offset) return fail(c, "boot_read: range exceeds buffer");
    if (bytes == 0) return 1;
    if (!hip_ok(c, hipMemcpyAsync(host, (char *)b->ptr + offset, bytes, hipMemcpyDeviceToHost, c->stream), "boot_read"))
        return 0;
    return hip_ok(c, hipStreamSynchronize(c->stream), "boot_read");
}

}  // extern "C"
