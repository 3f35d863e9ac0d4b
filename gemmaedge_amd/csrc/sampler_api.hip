// C ABI of the gfx950 sampling path (include/gemmaedge_sampler.h).
//
// Conventions follow the reference's accelerator layer where it has one:
// a cached availability probe (src/cuda_backend.cu:571-580), workspaces sized
// once and reused (src/cuda_backend.cu:388-425), and a status return instead of
// a C++ exception across the boundary. Unlike the reference there is no
// process-wide lock (src/cuda_backend.cu:513): a handle belongs to one stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/gemmaedge_sampler.h"
#include "sampler_internal.h"
#include "sampler_validate.h"

static_assert(ge::kPlanBlock == ge::kBlock && ge::kPlanMaxTopK == ge::kMaxTopK &&
                  ge::kPlanMaxChunks == ge::kMaxChunks && ge::kPlanMaxChunkLen == ge::kBlock * ge::kMaxEpt,
              "plan and kernel geometry");
static_assert(ge::kPlanStreamMaxChunks == ge::kStreamMaxChunks && ge::kStreamMaxChunks * 4 <= 64, "single-pass geometry");

struct ge_sampler {
    int device;
    int max_rows;
    int max_vocab;
    int max_history;
    uint32_t* tickets;
    uint64_t* slots;
    uint64_t* poll;  // greedy calls on small grids, zero at creation
    uint64_t* plists;  // single-pass kernel's candidate lists and call counts, zero at creation
    // Full-order path (bf16 rows with k > kMaxTopK); allocated when max_vocab > kMaxTopK.
    uint64_t* fo_items;
    float* fo_aux;
    uint32_t* fo_pre;
    uint64_t* fo_extras;
    uint32_t* fo_bitmap;
    uint32_t* fo_meta;
    uint32_t* fo_tiles;
    int64_t fo_tiles_words;
    int64_t fo_items_stride;
    int64_t fo_capacity;
    int32_t fo_extras_cap;
    int64_t fo_bitmap_words;
};

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(GE_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

// Switches the calling thread to `device` for the lifetime of the object.
struct DeviceGuard {
    int prev = -1;
    bool ok = true;
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != device) ok = hipSetDevice(device) == hipSuccess;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

bool device_is_gfx950(int device) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return false;
    return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
}

constexpr int64_t kMaxChunkLen = static_cast<int64_t>(ge::kBlock) * ge::kMaxEpt;

}  // namespace

extern "C" {

const char* ge_sampler_last_error(void) { return g_last_error.c_str(); }

int ge_sampler_max_top_k(void) { return ge::kMaxTopK; }

int ge_sampler_available(void) {
    static int cached = -1;
    if (cached < 0) {
        int n = 0;
        int found = 0;
        if (hipGetDeviceCount(&n) == hipSuccess) {
            for (int d = 0; d < n && !found; ++d) found = device_is_gfx950(d) ? 1 : 0;
        }
        cached = found;
    }
    return cached;
}

int ge_sampler_create(int device, int max_rows, int max_vocab, int max_history, ge_sampler** out) {
    if (!out) return fail(GE_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (max_rows < 1 || max_vocab < 1 || max_history < 0)
        return fail(GE_ERR_INVALID_ARG, "max_rows=%d max_vocab=%d max_history=%d", max_rows,
                    max_vocab, max_history);
    if (static_cast<int64_t>(max_vocab) > kMaxChunkLen * ge::kMaxChunks)
        return fail(GE_ERR_CAPACITY, "max_vocab %d above %lld", max_vocab,
                    static_cast<long long>(kMaxChunkLen * ge::kMaxChunks));
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n)
        return fail(GE_ERR_NO_DEVICE, "device %d not present (%d devices)", device, n);
    if (!device_is_gfx950(device)) return fail(GE_ERR_NO_DEVICE, "device %d is not gfx950", device);
    DeviceGuard guard(device);
    if (!guard.ok) return fail(GE_ERR_DEVICE, "hipSetDevice(%d) failed", device);

    ge_sampler* s = new ge_sampler{};
    s->device = device;
    s->max_rows = max_rows;
    s->max_vocab = max_vocab;
    s->max_history = max_history;
    const size_t rows = static_cast<size_t>(max_rows);
    hipError_t e = hipSuccess;
    auto alloc = [&](void** p, size_t bytes) {
        if (e == hipSuccess) e = hipMalloc(p, bytes);
    };
    alloc(reinterpret_cast<void**>(&s->tickets), rows * sizeof(uint32_t));
    alloc(reinterpret_cast<void**>(&s->slots), rows * ge::kSlotWords * sizeof(uint64_t));
    alloc(reinterpret_cast<void**>(&s->poll), rows * ge::kPollStride * sizeof(uint64_t));
    alloc(reinterpret_cast<void**>(&s->plists), rows * ge::kPollRowWords * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMemset(s->tickets, 0, rows * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(s->poll, 0, rows * ge::kPollStride * sizeof(uint64_t));
    if (e == hipSuccess) e = hipMemset(s->plists, 0, rows * ge::kPollRowWords * sizeof(uint64_t));
    if (max_vocab > ge::kMaxTopK) {
        s->fo_items_stride = ge::fo_items_stride(max_history);
        s->fo_extras_cap = max_history < ge::kFoExtrasCap ? (max_history > 0 ? max_history : 1) : ge::kFoExtrasCap;
        s->fo_bitmap_words = (static_cast<int64_t>(max_vocab) + 31) / 32;
        // f32 full-order rows take V items each (16 B per item over the three
        // arrays): room for up to 256 of them per launch pair, one per CU.
        const size_t f32_rows = std::min<size_t>(rows, 256);
        const size_t items = std::max(rows * static_cast<size_t>(s->fo_items_stride),
                                      f32_rows * static_cast<size_t>(ge::fo_items_stride_f32(max_vocab)));
        s->fo_capacity = static_cast<int64_t>(items);
        const size_t words = rows * static_cast<size_t>(s->fo_bitmap_words);
        alloc(reinterpret_cast<void**>(&s->fo_items), items * sizeof(uint64_t));
        alloc(reinterpret_cast<void**>(&s->fo_aux), items * sizeof(float));
        alloc(reinterpret_cast<void**>(&s->fo_pre), items * sizeof(uint32_t));
        alloc(reinterpret_cast<void**>(&s->fo_extras), rows * static_cast<size_t>(s->fo_extras_cap) * sizeof(uint64_t));
        alloc(reinterpret_cast<void**>(&s->fo_bitmap), words * sizeof(uint32_t));
        alloc(reinterpret_cast<void**>(&s->fo_meta), rows * ge::kMetaWords * sizeof(uint32_t));
        // the many-workgroup f32 sort: per-tile counts for the same 256 rows
        s->fo_tiles_words = static_cast<int64_t>(f32_rows) * ge::fo_tile_words(ge::fo_split_tiles(max_vocab));
        alloc(reinterpret_cast<void**>(&s->fo_tiles), static_cast<size_t>(s->fo_tiles_words) * sizeof(uint32_t));
        if (e == hipSuccess) e = hipMemset(s->fo_bitmap, 0, words * sizeof(uint32_t));
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        ge_sampler_destroy(s);
        return hip_fail(e, "ge_sampler_create");
    }
    *out = s;
    return GE_OK;
}

void ge_sampler_destroy(ge_sampler* s) {
    if (!s) return;
    DeviceGuard guard(s->device);
    (void)hipFree(s->tickets);
    (void)hipFree(s->slots);
    (void)hipFree(s->poll);
    (void)hipFree(s->plists);
    (void)hipFree(s->fo_items);
    (void)hipFree(s->fo_aux);
    (void)hipFree(s->fo_pre);
    (void)hipFree(s->fo_extras);
    (void)hipFree(s->fo_bitmap);
    (void)hipFree(s->fo_meta);
    (void)hipFree(s->fo_tiles);
    delete s;
}

}  // extern "C"

namespace {

// The workspace one call runs on: a handle's buffers (ge_sample) or the
// static array (ge_sample_noalloc, which has no full-order workspace).
struct Workspace {
    int device;
    int max_rows;
    int max_vocab;
    int max_history;
    uint32_t* tickets;
    uint64_t* slots;
    uint64_t* poll;  // NULL: greedy rows take tickets
    uint64_t* plists;  // NULL: no single-pass kernel
    uint64_t* fo_items;
    float* fo_aux;
    uint32_t* fo_pre;
    uint64_t* fo_extras;
    uint32_t* fo_bitmap;
    uint32_t* fo_meta;
    uint32_t* fo_tiles;
    int64_t fo_tiles_words;
    int64_t fo_items_stride;
    int64_t fo_capacity;
    int32_t fo_extras_cap;
    int64_t fo_bitmap_words;
};

// Validates the arguments against the workspace and launches the kernels on
// `stream` (the caller has made ws.device current).
int sample_on(const Workspace& ws, void* stream, const ge_sample_args& x) {
    ge::CallPlan plan{};
    char msg[256];
    const int rc = ge::plan_call(
        x, ge::CallCapacity{ws.max_rows, ws.max_vocab, ws.fo_items != nullptr, ws.plists != nullptr}, plan, msg,
        sizeof(msg));
    if (rc != GE_OK) return fail(rc, "%s", msg);
    const bool run_select = plan.run_select;
    const bool run_full = plan.run_full;
    const int ept = plan.ept;
    const int chunk_len = ge::kBlock * ept;
    const int cpr = plan.cpr;
    const bool vec_ok = plan.vec_ok;

    ge::DevArgs a{};
    a.logits = x.logits;
    a.dtype = x.dtype;
    a.rows = x.rows;
    a.vocab = x.vocab;
    a.row_stride = x.row_stride;
    a.params = x.params;
    a.row_params = x.row_params;
    a.history = x.history;
    a.history_offsets = x.history_offsets;
    a.ring = x.ring;
    a.ring_len = x.ring_len;
    a.ring_capacity = x.ring_capacity;
    a.uniforms = x.uniforms;
    a.tokens = x.tokens_out;
    a.probs = x.probs_out;
    a.flags = x.flags_out;
    a.stop_tokens = x.n_stop > 0 ? x.stop_tokens : nullptr;
    a.n_stop = x.n_stop;
    a.stop_mode = x.stop_mode;
    a.done = x.done;
    a.tickets = ws.tickets;
    a.slots = ws.slots;
    // Greedy chunks publish polled words when every workgroup of the launch
    // can be resident at once and indices fit the word's 24-bit field.
    const bool poll = plan.run_greedy && ws.poll && cpr <= ge::kPollChunks &&
                      static_cast<int64_t>(x.rows) * cpr <= ge::kPollMaxBlocks && x.vocab < (1 << 24);
    a.poll = poll ? ws.poll : nullptr;
    a.plists = plan.run_stream ? ws.plists : nullptr;
    a.cpr = cpr;
    a.chunk_len = chunk_len;
    a.vec_ok = vec_ok ? 1 : 0;
    a.fo_items = ws.fo_items;
    a.fo_aux = ws.fo_aux;
    a.fo_pre = ws.fo_pre;
    a.fo_extras = ws.fo_extras;
    a.fo_bitmap = ws.fo_bitmap;
    a.fo_meta = ws.fo_meta;
    a.fo_tiles = ws.fo_tiles;
    a.fo_tiles_words = ws.fo_tiles_words;
    a.fo_items_stride = ws.fo_items_stride;
    a.fo_extras_cap = ws.fo_extras_cap;
    a.fo_bitmap_words = ws.fo_bitmap_words;
    a.fo_capacity = ws.fo_capacity;

    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (plan.run_greedy) {
        const hipError_t e = ge::launch_greedy(a, st, ept);
        if (e != hipSuccess) return hip_fail(e, "launch (greedy)");
    }
    if (plan.run_stream) {
        const hipError_t e = ge::launch_stream(a, st);
        if (e != hipSuccess) return hip_fail(e, "launch (single pass)");
    } else if (run_select) {
        const hipError_t e = ge::launch_select(a, st, ept);
        if (e != hipSuccess) return hip_fail(e, "launch");
    }
    if (run_full) {
        // A bf16 row may hold more unique penalised ids than the extras
        // workspace when its history can be that long: a device ring's
        // capacity, else the handle's max_history.
        const int64_t hmax = x.ring ? std::max<int64_t>(x.ring_capacity, ws.max_history) : ws.max_history;
        const bool overflow = x.dtype == GE_DTYPE_BF16 && hmax > ws.fo_extras_cap;
        const hipError_t e = ge::launch_full_order(a, st, overflow);
        if (e != hipSuccess) return hip_fail(e, "launch (full order)");
    }
    return GE_OK;
}

// ---- allocation-free entry point ---------------------------------------------
//
// The selection path's workspace for GE_NOALLOC_MAX_ROWS rows in a file-scope
// device array: u32 tickets (zero between calls) in the first kTicketBytes,
// then kSlotWords u64 list words per row. Each GPU the library runs on holds
// its own copy until the process ends. Host code uses the array only through
// the address hipGetSymbolAddress returns for the current device (its name is
// a host-side stand-in, not a device address).
constexpr size_t kTicketBytes = 4096;
static_assert(GE_NOALLOC_MAX_ROWS * sizeof(uint32_t) <= kTicketBytes, "ticket area");
constexpr size_t kScratchBytes =
    kTicketBytes + static_cast<size_t>(GE_NOALLOC_MAX_ROWS) * ge::kSlotWords * sizeof(uint64_t);
static_assert(kScratchBytes == GE_NOALLOC_SCRATCH_BYTES, "GE_NOALLOC_SCRATCH_BYTES");
static __device__ __align__(256) uint64_t scratch[kScratchBytes / sizeof(uint64_t)];

constexpr int kMaxDevices = 64;

__global__ void clear_words(uint32_t* p, int n) {
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < n) p[i] = 0u;
}

// The array's address on `device` (current), found once per device; its
// ticket area is cleared on `stream` the first time (a kernel, not a memset).
// The device's gfx950 check is made at that first call too, not per call.
int scratch_on(int device, hipStream_t stream, void** out) {
    static std::mutex mu;
    static void* ptr[kMaxDevices] = {};
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[device]) {
        if (!device_is_gfx950(device)) return fail(GE_ERR_NO_DEVICE, "device %d is not gfx950", device);
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(GE_ERR_DEVICE, "hipGetSymbolAddress(scratch) returned NULL");
        constexpr int kWords = static_cast<int>(kTicketBytes / sizeof(uint32_t));
        hipLaunchKernelGGL(clear_words, dim3((kWords + 255) / 256), dim3(256), 0, stream,
                           static_cast<uint32_t*>(p), kWords);
        const hipError_t e2 = hipGetLastError();
        if (e2 != hipSuccess) return hip_fail(e2, "clear scratch tickets");
        ptr[device] = p;
    }
    *out = ptr[device];
    return GE_OK;
}

}  // namespace

extern "C" {

int ge_sample(ge_sampler* s, void* stream, const ge_sample_args* args) {
    if (!s || !args) return fail(GE_ERR_INVALID_ARG, "sampler or args is NULL");
    DeviceGuard guard(s->device);
    if (!guard.ok) return fail(GE_ERR_DEVICE, "hipSetDevice(%d) failed", s->device);
    Workspace ws{};
    ws.device = s->device;
    ws.max_rows = s->max_rows;
    ws.max_vocab = s->max_vocab;
    ws.max_history = s->max_history;
    ws.tickets = s->tickets;
    ws.slots = s->slots;
    ws.poll = s->poll;
    ws.plists = s->plists;
    ws.fo_items = s->fo_items;
    ws.fo_aux = s->fo_aux;
    ws.fo_pre = s->fo_pre;
    ws.fo_extras = s->fo_extras;
    ws.fo_bitmap = s->fo_bitmap;
    ws.fo_meta = s->fo_meta;
    ws.fo_tiles = s->fo_tiles;
    ws.fo_tiles_words = s->fo_tiles_words;
    ws.fo_items_stride = s->fo_items_stride;
    ws.fo_capacity = s->fo_capacity;
    ws.fo_extras_cap = s->fo_extras_cap;
    ws.fo_bitmap_words = s->fo_bitmap_words;
    return sample_on(ws, stream, *args);
}

int ge_sample_noalloc(void* stream, const ge_sample_args* args) {
    if (!args) return fail(GE_ERR_INVALID_ARG, "args is NULL");
    if (args->rows > GE_NOALLOC_MAX_ROWS)
        return fail(GE_ERR_CAPACITY, "rows %d above GE_NOALLOC_MAX_ROWS (%d)", args->rows, GE_NOALLOC_MAX_ROWS);
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices)
        return fail(GE_ERR_NO_DEVICE, "no current device");
    void* p = nullptr;
    const int rc = scratch_on(device, static_cast<hipStream_t>(stream), &p);
    if (rc != GE_OK) return rc;
    Workspace ws{};
    ws.device = device;
    ws.max_rows = GE_NOALLOC_MAX_ROWS;
    ws.max_vocab = static_cast<int>(kMaxChunkLen * ge::kMaxChunks);
    ws.tickets = static_cast<uint32_t*>(p);
    ws.slots = reinterpret_cast<uint64_t*>(static_cast<char*>(p) + kTicketBytes);
    return sample_on(ws, stream, *args);
}

}  // extern "C"
