// Host side of the device boundary: the Safety Governor, Governor-reserved allocations and the
// matvec accelerator with device residency (include/vastloom_hip.h). Plain C++; the only device
// work is in the HIP backend at the end of this file, which calls the kernels of vl_kernels.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/vastloom_hip.h"
#include "vl_error.h"
#include "vl_kernels.h"
#include "vl_layout.h"

using vl::fail;

// ------------------------------------------------------------------------------------------
// Governor (src/safety/resource_governor.cpp).
// ------------------------------------------------------------------------------------------

struct vl_governor {
    struct Held {
        uint32_t kind;
        uint64_t bytes;
    };
    vl_resource_limits limits{};
    mutable std::mutex mutex;
    uint64_t reserved[4]{};
    uint32_t state = VL_STATE_NORMAL;
    uint32_t recovery_counter = 0;
    uint64_t next_id = 1;
    std::unordered_map<uint64_t, Held> held;

    uint64_t limit_for(uint32_t kind) const {
        switch (kind) {
            case VL_KIND_RAM: return limits.ram_hard_limit;
            case VL_KIND_VRAM: return limits.vram_hard_limit;
            case VL_KIND_STAGING: return limits.staging_hard_limit;
            case VL_KIND_SCRATCH: return limits.scratch_hard_limit;
            default: return 0;
        }
    }
};

namespace {

const char* kind_name(uint32_t kind) {
    switch (kind) {
        case VL_KIND_RAM: return "ram";
        case VL_KIND_VRAM: return "vram";
        case VL_KIND_STAGING: return "staging";
        case VL_KIND_SCRATCH: return "scratch";
        default: return "unknown";
    }
}

const char* state_name(uint32_t state) {
    switch (state) {
        case VL_STATE_NORMAL: return "normal";
        case VL_STATE_PRESSURE: return "pressure";
        case VL_STATE_CRITICAL: return "critical";
        default: return "emergency";
    }
}

uint32_t ratio_state(double ratio, const vl_resource_limits& l) {
    return ratio >= l.critical_ratio ? VL_STATE_CRITICAL
         : ratio >= l.pressure_ratio ? VL_STATE_PRESSURE
                                     : VL_STATE_NORMAL;
}

// Native Governor behind vl_governor_ops.
int ops_reserve(void* ctx, uint32_t kind, uint64_t bytes, const char* tag, uint64_t* id) {
    return vl_governor_try_reserve(static_cast<vl_governor*>(ctx), kind, bytes, tag, id);
}
void ops_release(void* ctx, uint64_t id) { vl_governor_release(static_cast<vl_governor*>(ctx), id); }
void ops_abandon(void* ctx, uint64_t id) { vl_governor_abandon(static_cast<vl_governor*>(ctx), id); }

bool ops_valid(const vl_governor_ops* g) {
    return g && g->try_reserve && g->release && g->abandon;
}

}  // namespace

extern "C" {

void vl_resource_limits_default(vl_resource_limits* l) {
    if (!l) return;
    std::memset(l, 0, sizeof *l);
    l->minimum_system_ram_available = 2ull << 30;
    l->minimum_storage_available = 20ull << 30;
    l->pressure_ratio = 0.82;
    l->critical_ratio = 0.93;
    l->recovery_samples = 3;
}

int vl_vram_hard_limit(uint64_t total_vram_bytes, uint64_t free_vram_bytes, uint64_t* limit) {
    if (!limit) return fail(VL_INVALID_ARGUMENT, "limit is null");
    constexpr uint64_t kGiB = 1ull << 30;
    uint64_t v = 0;
    if (free_vram_bytes > kGiB) {
        const uint64_t pct = (uint64_t)((long double)total_vram_bytes * (long double)0.80);
        v = pct < free_vram_bytes - kGiB ? pct : free_vram_bytes - kGiB;
    }
    *limit = v;
    return VL_OK;
}

int vl_governor_create(const vl_resource_limits* limits, vl_governor** out) {
    if (!limits || !out) return fail(VL_INVALID_ARGUMENT, "null argument");
    vl_governor* g = new (std::nothrow) vl_governor;
    if (!g) return fail(VL_RESOURCE_EXHAUSTED, "unable to allocate the governor");
    g->limits = *limits;
    // ResourceGovernor::ResourceGovernor (resource_governor.cpp:58-62).
    g->limits.pressure_ratio = std::clamp(g->limits.pressure_ratio, 0.10, 0.99);
    g->limits.critical_ratio = std::clamp(g->limits.critical_ratio, g->limits.pressure_ratio + 0.01, 1.0);
    g->limits.recovery_samples = std::max(1u, g->limits.recovery_samples);
    *out = g;
    return VL_OK;
}

void vl_governor_destroy(vl_governor* g) { delete g; }

int vl_governor_try_reserve(vl_governor* g, uint32_t kind, uint64_t bytes, const char* tag,
                            uint64_t* id) {
    if (!g || !id) return fail(VL_INVALID_ARGUMENT, "null argument");
    const char* t = tag ? tag : "";
    if (kind > VL_KIND_SCRATCH) return fail(VL_INVALID_ARGUMENT, "unknown resource kind %u (%s)", kind, t);
    if (bytes == 0) return fail(VL_INVALID_ARGUMENT, "A zero-byte reservation is not allowed (%s)", t);
    std::lock_guard<std::mutex> lock(g->mutex);
    if (g->state == VL_STATE_CRITICAL || g->state == VL_STATE_EMERGENCY)
        return fail(VL_RESOURCE_EXHAUSTED, "Safety governor rejected new work in %s state (%s)",
                    state_name(g->state), t);
    const uint64_t limit = g->limit_for(kind);
    if (limit == 0 || bytes > limit || g->reserved[kind] > limit - bytes)
        return fail(VL_RESOURCE_EXHAUSTED, "Reservation would exceed the hard %s budget (%s)",
                    kind_name(kind), t);
    if (kind != VL_KIND_VRAM && g->limits.host_memory_hard_limit != 0) {
        uint64_t remaining = g->limits.host_memory_hard_limit;
        for (uint32_t hk : {VL_KIND_RAM, VL_KIND_STAGING, VL_KIND_SCRATCH}) {
            if (g->reserved[hk] > remaining)
                return fail(VL_INTEGRITY_ERROR,
                            "Host-memory reservations exceed their aggregate hard limit (%s)", t);
            remaining -= g->reserved[hk];
        }
        if (bytes > remaining)
            return fail(VL_RESOURCE_EXHAUSTED,
                        "Reservation would exceed the aggregate host-memory budget (%s)", t);
    }
    try {
        const uint64_t rid = g->next_id++;
        g->held.emplace(rid, vl_governor::Held{kind, bytes});
        g->reserved[kind] += bytes;
        *id = rid;
    } catch (const std::bad_alloc&) {
        return fail(VL_RESOURCE_EXHAUSTED, "unable to record a reservation (%s)", t);
    }
    return VL_OK;
}

int vl_governor_release(vl_governor* g, uint64_t id) {
    if (!g) return fail(VL_INVALID_ARGUMENT, "null governor");
    std::lock_guard<std::mutex> lock(g->mutex);
    auto it = g->held.find(id);
    if (it == g->held.end()) return fail(VL_NOT_FOUND, "no reservation %llu", (unsigned long long)id);
    uint64_t& r = g->reserved[it->second.kind];
    r = it->second.bytes >= r ? 0 : r - it->second.bytes;
    g->held.erase(it);
    return VL_OK;
}

int vl_governor_abandon(vl_governor* g, uint64_t id) {
    if (!g) return fail(VL_INVALID_ARGUMENT, "null governor");
    std::lock_guard<std::mutex> lock(g->mutex);
    auto it = g->held.find(id);
    if (it == g->held.end()) return fail(VL_NOT_FOUND, "no reservation %llu", (unsigned long long)id);
    g->held.erase(it);  // the bytes stay in reserved[]
    return VL_OK;
}

int vl_governor_update_pressure(vl_governor* g, const vl_runtime_pressure* p, uint32_t* state) {
    if (!g || !p) return fail(VL_INVALID_ARGUMENT, "null argument");
    std::lock_guard<std::mutex> lock(g->mutex);
    const vl_resource_limits& l = g->limits;
    uint32_t raw = VL_STATE_NORMAL;
    const uint64_t hard[4] = {l.ram_hard_limit, l.vram_hard_limit, l.staging_hard_limit, l.scratch_hard_limit};
    for (uint32_t k = 0; k < 4; ++k)
        if (hard[k] != 0) raw = std::max(raw, ratio_state((double)g->reserved[k] / (double)hard[k], l));
    if (l.host_memory_hard_limit != 0) {
        uint64_t host = 0;
        for (uint32_t hk : {VL_KIND_RAM, VL_KIND_STAGING, VL_KIND_SCRATCH}) {
            const uint64_t r = g->reserved[hk];
            host = r > l.host_memory_hard_limit - host ? l.host_memory_hard_limit : host + r;
        }
        raw = std::max(raw, ratio_state((double)host / (double)l.host_memory_hard_limit, l));
    }
    const auto reserve_state = [&raw](uint64_t avail, uint64_t minimum) {
        if (avail <= minimum / 4u) raw = VL_STATE_EMERGENCY;
        else if (avail <= minimum) raw = std::max(raw, (uint32_t)VL_STATE_CRITICAL);
        else if (avail <= minimum * 2u) raw = std::max(raw, (uint32_t)VL_STATE_PRESSURE);
    };
    reserve_state(p->system_ram_available, l.minimum_system_ram_available);
    reserve_state(p->storage_available, l.minimum_storage_available);
    if (raw > g->state) {
        g->state = raw;
        g->recovery_counter = 0;
    } else if (raw < g->state) {
        if (++g->recovery_counter >= l.recovery_samples) {
            g->state -= 1;
            g->recovery_counter = 0;
        }
    } else {
        g->recovery_counter = 0;
    }
    if (state) *state = g->state;
    return VL_OK;
}

int vl_governor_snapshot_get(const vl_governor* g, vl_governor_snapshot* out) {
    if (!g || !out) return fail(VL_INVALID_ARGUMENT, "null argument");
    std::lock_guard<std::mutex> lock(g->mutex);
    out->state = g->state;
    out->recovery_counter = g->recovery_counter;
    for (int k = 0; k < 4; ++k) out->reserved[k] = g->reserved[k];
    return VL_OK;
}

vl_governor_ops vl_governor_as_ops(vl_governor* g) {
    vl_governor_ops ops;
    ops.ctx = g;
    ops.try_reserve = ops_reserve;
    ops.release = ops_release;
    ops.abandon = ops_abandon;
    return ops;
}

}  // extern "C"

// ------------------------------------------------------------------------------------------
// Governed allocations (CudaDriver::allocate / CudaAllocation, src/cuda/cuda_driver.cpp).
// ------------------------------------------------------------------------------------------

struct vl_buffer {
    vl_governor_ops gov;
    uint64_t reservation;
    uint32_t kind;
    int device;
    void* ptr;
    uint64_t bytes;
};

namespace {

constexpr size_t kMaxTagBytes = 1024;

// Buffers whose memory could not be released: kept (and their bytes kept charged) until exit.
std::mutex g_quarantine_mutex;
std::vector<vl_buffer*>* g_quarantine = nullptr;

void quarantine(vl_buffer* b) {
    std::lock_guard<std::mutex> lock(g_quarantine_mutex);
    try {
        if (!g_quarantine) g_quarantine = new std::vector<vl_buffer*>;
        g_quarantine->push_back(b);
    } catch (const std::bad_alloc&) {
        // The handle leaks either way; nothing more to do.
    }
}

struct DeviceGuard {
    int saved = -1;
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&saved) != hipSuccess) saved = -1;
        if (saved != device) (void)hipSetDevice(device);
    }
    ~DeviceGuard() {
        if (saved >= 0) (void)hipSetDevice(saved);
    }
};

int hip_free_memory(int device, uint64_t* free_bytes) {
    DeviceGuard guard(device);
    size_t f = 0, t = 0;
    const hipError_t e = hipMemGetInfo(&f, &t);
    if (e != hipSuccess) return fail(VL_INTERNAL_ERROR, "hipMemGetInfo: %s", hipGetErrorString(e));
    *free_bytes = f;
    return VL_OK;
}

int hip_allocate(uint32_t kind, int device, uint64_t bytes, void** ptr) {
    DeviceGuard guard(device);
    hipError_t e;
    if (kind == VL_KIND_STAGING) e = hipHostMalloc(ptr, bytes, hipHostMallocDefault);
    else e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        *ptr = nullptr;
        return fail(VL_RESOURCE_EXHAUSTED, "%s of %llu bytes failed: %s",
                    kind == VL_KIND_STAGING ? "hipHostMalloc" : "hipMalloc",
                    (unsigned long long)bytes, hipGetErrorString(e));
    }
    return VL_OK;
}

int hip_release(uint32_t kind, int device, void* ptr) {
    DeviceGuard guard(device);
    const hipError_t e = kind == VL_KIND_STAGING ? hipHostFree(ptr) : hipFree(ptr);
    if (e != hipSuccess) return fail(VL_INTERNAL_ERROR, "release failed: %s", hipGetErrorString(e));
    return VL_OK;
}

}  // namespace

extern "C" {

int vl_buffer_alloc(const vl_governor_ops* gov, uint32_t kind, int device, uint64_t bytes,
                    uint64_t min_free_after, const char* tag, vl_buffer** out) {
    if (!out) return fail(VL_INVALID_ARGUMENT, "out is null");
    *out = nullptr;
    if (!ops_valid(gov)) return fail(VL_INVALID_ARGUMENT, "a governor is required");
    if (kind != VL_KIND_VRAM && kind != VL_KIND_STAGING)
        return fail(VL_INVALID_ARGUMENT, "buffers are device (vram) or pinned host (staging) memory");
    if (device < 0) return fail(VL_INVALID_ARGUMENT, "device ordinal cannot be negative");
    if (bytes == 0) return fail(VL_INVALID_ARGUMENT, "allocation size cannot be zero");
    const size_t tl = tag ? std::strlen(tag) : 0;
    if (tl == 0 || tl > kMaxTagBytes) return fail(VL_INVALID_ARGUMENT, "allocation tag must contain 1 to 1024 bytes");
    uint64_t rid = 0;
    int rc = gov->try_reserve(gov->ctx, kind, bytes, tag, &rid);
    if (rc != VL_OK) return rc;
    if (kind == VL_KIND_VRAM) {
        uint64_t free_bytes = 0;
        rc = hip_free_memory(device, &free_bytes);
        if (rc == VL_OK && (free_bytes < bytes || free_bytes - bytes < min_free_after))
            rc = fail(VL_RESOURCE_EXHAUSTED, "allocation of %llu bytes would leave less than %llu bytes free (%s)",
                      (unsigned long long)bytes, (unsigned long long)min_free_after, tag);
        if (rc != VL_OK) {
            gov->release(gov->ctx, rid);
            return rc;
        }
    }
    void* p = nullptr;
    rc = hip_allocate(kind, device, bytes, &p);
    if (rc != VL_OK) {
        gov->release(gov->ctx, rid);
        return rc;
    }
    vl_buffer* b = new (std::nothrow) vl_buffer{*gov, rid, kind, device, p, bytes};
    if (!b) {
        if (hip_release(kind, device, p) == VL_OK) gov->release(gov->ctx, rid);
        else gov->abandon(gov->ctx, rid);
        return fail(VL_RESOURCE_EXHAUSTED, "unable to allocate a buffer handle");
    }
    *out = b;
    return VL_OK;
}

void* vl_buffer_ptr(const vl_buffer* b) { return b ? b->ptr : nullptr; }
uint64_t vl_buffer_bytes(const vl_buffer* b) { return b ? b->bytes : 0; }

int vl_buffer_free(vl_buffer* b) {
    if (!b) return VL_OK;
    const int rc = hip_release(b->kind, b->device, b->ptr);
    if (rc != VL_OK) {
        // The memory may still be live: keep its bytes charged and never hand it out again.
        b->gov.abandon(b->gov.ctx, b->reservation);
        quarantine(b);
        return rc;
    }
    b->gov.release(b->gov.ctx, b->reservation);
    delete b;
    return VL_OK;
}

}  // extern "C"

// ------------------------------------------------------------------------------------------
// HIP backend of the accelerator.
// ------------------------------------------------------------------------------------------

namespace {

struct HipBackend {
    int device = 0;
    hipStream_t compute = nullptr;  // packs and matvecs
    hipStream_t copy = nullptr;     // host -> device uploads
    hipEvent_t h2d_done[2]{};       // slot's copy finished: its pinned staging is free again
    hipEvent_t pack_done[2]{};      // slot's pack finished: its device scratch is free again
    bool used[2]{false, false};
    uint32_t blocks = 0;
};

int hb_free_memory(void* ctx, int device, uint64_t* free_bytes) {
    (void)ctx;
    return hip_free_memory(device, free_bytes);
}

int hb_allocate(void* ctx, uint32_t kind, int device, uint64_t bytes, void** ptr) {
    (void)ctx;
    return hip_allocate(kind, device, bytes, ptr);
}

int hb_release(void* ctx, uint32_t kind, void* ptr) {
    return hip_release(kind, static_cast<HipBackend*>(ctx)->device, ptr);
}

int hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return VL_OK;
    return fail(VL_INTERNAL_ERROR, "%s: %s", what, hipGetErrorString(e));
}

// Row ranges of the GGUF matrix go host -> pinned slot (CPU copy) -> device scratch slot
// (hipMemcpyAsync on the copy stream) -> tiled form (pack on the compute stream), two slots
// alternating so that the CPU copy, the DMA and the pack of consecutive ranges overlap.
int hb_upload(void* ctx, uint32_t type, uint64_t rows, uint64_t cols, const void* gguf, void* tiled,
              void* staging, void* scratch, uint64_t staging_bytes) {
    HipBackend* hb = static_cast<HipBackend*>(ctx);
    DeviceGuard guard(hb->device);
    vl_tiled_layout L;
    if (!vl_make_layout(type, (uint32_t)rows, (uint32_t)cols, &L)) return fail(VL_UNSUPPORTED, "no layout");
    const uint64_t row_bytes = (uint64_t)(cols / L.block_elements) * L.block_bytes;
    const uint64_t slot = staging_bytes / 2u;
    uint64_t chunk_rows = slot / row_bytes / 32u * 32u;
    if (chunk_rows == 0) return fail(VL_RESOURCE_EXHAUSTED, "staging slots hold fewer than 32 rows");
    const uint8_t* src = static_cast<const uint8_t*>(gguf);
    uint8_t* pin = static_cast<uint8_t*>(staging);
    uint8_t* dev = static_cast<uint8_t*>(scratch);
    int rc = VL_OK;
    uint32_t i = 0;
    for (uint64_t r0 = 0; r0 < L.rows_padded && rc == VL_OK; r0 += chunk_rows, ++i) {
        const uint64_t r1 = std::min<uint64_t>(r0 + chunk_rows, L.rows_padded);
        const uint64_t data_rows = r0 < rows ? std::min<uint64_t>(r1, rows) - r0 : 0;
        const uint64_t nbytes = data_rows * row_bytes;
        const uint32_t s = i & 1u;
        if (hb->used[s]) {
            rc = hip_check(hipEventSynchronize(hb->h2d_done[s]), "hipEventSynchronize");
            if (rc == VL_OK) rc = hip_check(hipStreamWaitEvent(hb->copy, hb->pack_done[s], 0), "hipStreamWaitEvent");
            if (rc != VL_OK) break;
        }
        if (nbytes) {
            std::memcpy(pin + s * slot, src + r0 * row_bytes, nbytes);
            rc = hip_check(hipMemcpyAsync(dev + s * slot, pin + s * slot, nbytes, hipMemcpyHostToDevice, hb->copy),
                           "hipMemcpyAsync");
        }
        if (rc == VL_OK) rc = hip_check(hipEventRecord(hb->h2d_done[s], hb->copy), "hipEventRecord");
        if (rc == VL_OK) rc = hip_check(hipStreamWaitEvent(hb->compute, hb->h2d_done[s], 0), "hipStreamWaitEvent");
        if (rc == VL_OK)
            rc = hip_check(vl::launch_pack_rows(L, dev + s * slot, static_cast<uint8_t*>(tiled), (uint32_t)r0,
                                                (uint32_t)r1, hb->compute),
                           "pack");
        if (rc == VL_OK) rc = hip_check(hipEventRecord(hb->pack_done[s], hb->compute), "hipEventRecord");
        hb->used[s] = true;
    }
    return rc;
}

// x, then y, then the matvec workspace, each 256-byte aligned.
struct IoLayout {
    uint64_t x, y, ws, ws_bytes, bytes;
};

int io_layout(HipBackend* hb, uint32_t type, uint64_t rows, uint64_t cols, IoLayout* io) {
    const auto al = [](uint64_t v) { return (v + 255u) & ~uint64_t(255); };
    io->ws_bytes = vl::matvec_workspace_bytes(type, (uint32_t)rows, (uint32_t)cols, 1u, hb->blocks);
    io->x = 0;
    io->y = al(cols * 4u);
    io->ws = io->y + al(rows * 4u);
    io->bytes = io->ws + al(io->ws_bytes);
    return VL_OK;
}

int hb_io_bytes(void* ctx, uint32_t type, uint64_t rows, uint64_t cols, uint64_t* bytes) {
    IoLayout io;
    io_layout(static_cast<HipBackend*>(ctx), type, rows, cols, &io);
    *bytes = io.bytes;
    return VL_OK;
}

int hb_matvec(void* ctx, uint32_t type, uint64_t rows, uint64_t cols, const void* tiled,
              const float* x, float* y, void* io_ptr, uint64_t io_bytes) {
    HipBackend* hb = static_cast<HipBackend*>(ctx);
    DeviceGuard guard(hb->device);
    vl_tiled_layout L;
    if (!vl_make_layout(type, (uint32_t)rows, (uint32_t)cols, &L)) return fail(VL_UNSUPPORTED, "no layout");
    IoLayout io;
    io_layout(hb, type, rows, cols, &io);
    if (io.bytes > io_bytes) return fail(VL_INTERNAL_ERROR, "matvec buffer too small");
    uint8_t* base = static_cast<uint8_t*>(io_ptr);
    float* xd = reinterpret_cast<float*>(base + io.x);
    float* yd = reinterpret_cast<float*>(base + io.y);
    uint8_t* ws = base + io.ws;
    int rc = hip_check(hipMemcpyAsync(xd, x, cols * 4u, hipMemcpyHostToDevice, hb->compute), "hipMemcpyAsync");
    if (rc == VL_OK)
        rc = hip_check(vl::launch_matvec(L, static_cast<const uint8_t*>(tiled), xd, 1u, yd, ws, hb->blocks,
                                         hb->compute),
                       "matvec");
    uint32_t status = 0;
    if (rc == VL_OK)
        rc = hip_check(hipMemcpyAsync(&status, ws, 4u, hipMemcpyDeviceToHost, hb->compute), "hipMemcpyAsync");
    std::vector<float> tmp;
    if (rc == VL_OK) {
        try {
            tmp.resize(rows);
        } catch (const std::bad_alloc&) {
            rc = fail(VL_RESOURCE_EXHAUSTED, "matvec output staging");
        }
    }
    if (rc == VL_OK)
        rc = hip_check(hipMemcpyAsync(tmp.data(), yd, rows * 4u, hipMemcpyDeviceToHost, hb->compute), "hipMemcpyAsync");
    if (rc == VL_OK) rc = hip_check(hipStreamSynchronize(hb->compute), "hipStreamSynchronize");
    if (rc != VL_OK) return rc;
    // The reference refuses non-finite inputs before and non-finite outputs after the product
    // (ggml_quantization.cpp:591-599, :808-813); the output stays untouched then.
    if (status & vl::kStatusNonFiniteInput) return fail(VL_INVALID_ARGUMENT, "matvec input contains a non-finite value");
    if (status & vl::kStatusNonFiniteOutput) return fail(VL_INVALID_ARGUMENT, "matvec produced a non-finite value");
    std::memcpy(y, tmp.data(), rows * 4u);
    return VL_OK;
}

HipBackend* hip_backend_create(int device, int* rc) {
    DeviceGuard guard(device);
    HipBackend* hb = new (std::nothrow) HipBackend;
    if (!hb) {
        *rc = fail(VL_RESOURCE_EXHAUSTED, "unable to allocate the HIP backend");
        return nullptr;
    }
    hb->device = device;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&hb->compute, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&hb->copy, hipStreamNonBlocking);
    for (int s = 0; s < 2 && e == hipSuccess; ++s) {
        e = hipEventCreateWithFlags(&hb->h2d_done[s], hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&hb->pack_done[s], hipEventDisableTiming);
    }
    if (e == hipSuccess) {
        hb->blocks = vl::stream_blocks();
        if (hb->blocks == 0) e = hipErrorNoDevice;
    }
    if (e != hipSuccess) {
        *rc = fail(VL_UNSUPPORTED, "HIP device %d is not usable: %s", device, hipGetErrorString(e));
        for (int s = 0; s < 2; ++s) {
            if (hb->h2d_done[s]) (void)hipEventDestroy(hb->h2d_done[s]);
            if (hb->pack_done[s]) (void)hipEventDestroy(hb->pack_done[s]);
        }
        if (hb->copy) (void)hipStreamDestroy(hb->copy);
        if (hb->compute) (void)hipStreamDestroy(hb->compute);
        delete hb;
        return nullptr;
    }
    *rc = VL_OK;
    return hb;
}

void hip_backend_destroy(HipBackend* hb) {
    if (!hb) return;
    DeviceGuard guard(hb->device);
    (void)hipStreamSynchronize(hb->copy);
    (void)hipStreamSynchronize(hb->compute);
    for (int s = 0; s < 2; ++s) {
        (void)hipEventDestroy(hb->h2d_done[s]);
        (void)hipEventDestroy(hb->pack_done[s]);
    }
    (void)hipStreamDestroy(hb->copy);
    (void)hipStreamDestroy(hb->compute);
    delete hb;
}

void hb_synchronize(HipBackend* hb) {
    DeviceGuard guard(hb->device);
    (void)hipStreamSynchronize(hb->copy);
    (void)hipStreamSynchronize(hb->compute);
}

}  // namespace

// ------------------------------------------------------------------------------------------
// Accelerator (src/cuda/cuda_matvec_accelerator.cpp:102-314).
// ------------------------------------------------------------------------------------------

struct vl_accel {
    struct Resident {
        void* tiled = nullptr;
        uint64_t reservation = 0;
        uint64_t total_bytes = 0;
        uint64_t matrix_bytes = 0;
        uint64_t last_used = 0;
        uint64_t rows = 0, cols = 0;
        uint32_t type = 0;
        bool recurring = false;
    };
    struct Held {  // a Governor-reserved device or pinned allocation
        void* ptr = nullptr;
        uint64_t reservation = 0;
        uint64_t bytes = 0;
    };
    vl_accel_options opt{};
    vl_governor_ops gov{};
    vl_accel_backend be{};
    HipBackend* hip = nullptr;  // owned when be is the HIP backend
    std::unordered_map<uint64_t, Resident> resident;
    uint64_t clock = 0;
    vl_accel_stats stats{};
    Held staging, scratch, io;
};

namespace {

bool has_kernel(uint32_t type) {
    return type == VL_GGML_Q8_0 || type == VL_GGML_IQ2_XXS || type == VL_GGML_IQ3_XXS ||
           type == VL_GGML_IQ1_S;
}

void count_declined_type(vl_accel_stats& st, uint32_t type) {
    for (uint32_t i = 0; i < VL_ACCEL_TYPE_SLOTS; ++i) {
        if (st.declined_by_type[i] != 0 && st.declined_type[i] == type) {
            ++st.declined_by_type[i];
            return;
        }
        if (st.declined_by_type[i] == 0) {
            st.declined_type[i] = type;
            st.declined_by_type[i] = 1;
            return;
        }
    }
    // More distinct types than slots: losing a statistic is not a reason to fail.
}

// Reserve, check the free-memory floor (device memory), allocate. A refusal returns
// VL_RESOURCE_EXHAUSTED with nothing held.
int acquire(vl_accel* a, uint32_t kind, uint64_t bytes, const char* tag, vl_accel::Held* h) {
    uint64_t rid = 0;
    int rc = a->gov.try_reserve(a->gov.ctx, kind, bytes, tag, &rid);
    if (rc != VL_OK) return rc;
    if (kind == VL_KIND_VRAM) {
        uint64_t free_bytes = 0;
        rc = a->be.free_memory(a->be.ctx, a->opt.device_ordinal, &free_bytes);
        if (rc == VL_OK && (free_bytes < bytes || free_bytes - bytes < a->opt.minimum_free_vram_after))
            rc = fail(VL_RESOURCE_EXHAUSTED, "%s: too little free device memory", tag);
        if (rc != VL_OK) {
            a->gov.release(a->gov.ctx, rid);
            return rc;
        }
    }
    void* p = nullptr;
    rc = a->be.allocate(a->be.ctx, kind, a->opt.device_ordinal, bytes, &p);
    if (rc != VL_OK || !p) {
        a->gov.release(a->gov.ctx, rid);
        return rc != VL_OK ? rc : fail(VL_RESOURCE_EXHAUSTED, "%s: allocation failed", tag);
    }
    h->ptr = p;
    h->reservation = rid;
    h->bytes = bytes;
    return VL_OK;
}

// Frees and returns the bytes; a failed free keeps the bytes charged and forgets the memory.
int give_back(vl_accel* a, uint32_t kind, vl_accel::Held* h) {
    if (!h->ptr) return VL_OK;
    const int rc = a->be.release(a->be.ctx, kind, h->ptr);
    if (rc != VL_OK) a->gov.abandon(a->gov.ctx, h->reservation);
    else a->gov.release(a->gov.ctx, h->reservation);
    h->ptr = nullptr;
    h->reservation = 0;
    h->bytes = 0;
    return rc;
}

int release_resident(vl_accel* a, vl_accel::Resident& r) {
    vl_accel::Held h{r.tiled, r.reservation, r.total_bytes};
    r.tiled = nullptr;
    return give_back(a, VL_KIND_VRAM, &h);
}

// The resident entry for this matrix, uploading it on first sight; *out = nullptr means the
// accelerator declines it (CudaMatvecAccelerator::ensure_resident).
int ensure_resident(vl_accel* a, const vl_packed_matrix& m, vl_accel::Resident** out) {
    *out = nullptr;
    if (a->opt.experts_only && m.recurring) {
        ++a->stats.declined_recurring;
        return VL_OK;
    }
    if (!has_kernel(m.ggml_type)) {
        count_declined_type(a->stats, m.ggml_type);
        return VL_OK;
    }
    uint32_t be = 0, bb = 0;
    vl_block_shape(m.ggml_type, &be, &bb);
    if (m.rows == 0 || m.storage_columns == 0 || m.storage_columns % be != 0) return VL_OK;
    if (m.cache_identity == 0) return VL_OK;
    auto it = a->resident.find(m.cache_identity);
    if (it != a->resident.end()) {
        it->second.last_used = ++a->clock;
        *out = &it->second;
        return VL_OK;
    }
    if (!m.encoded) return fail(VL_INVALID_ARGUMENT, "matrix %llu has no payload", (unsigned long long)m.cache_identity);
    vl_tiled_layout L;
    if (m.rows > 0x7fffffffu || m.storage_columns > 0x7fffffffu ||
        !vl_make_layout(m.ggml_type, (uint32_t)m.rows, (uint32_t)m.storage_columns, &L))
        return VL_OK;
    if (m.encoded_bytes != L.gguf_bytes) return VL_OK;
    const uint64_t total = L.bytes;
    if (total > a->opt.maximum_resident_bytes) return VL_OK;
    // Room: evict what will not recur first, then the least recently used.
    while ((a->stats.resident_bytes + total > a->opt.maximum_resident_bytes ||
            a->resident.size() >= a->opt.maximum_matrices) &&
           !a->resident.empty()) {
        auto victim = std::min_element(a->resident.begin(), a->resident.end(),
                                       [](const auto& l, const auto& r) {
                                           if (l.second.recurring != r.second.recurring) return !l.second.recurring;
                                           return l.second.last_used < r.second.last_used;
                                       });
        const uint64_t reclaimed = victim->second.total_bytes;
        const int rc = release_resident(a, victim->second);
        a->resident.erase(victim);
        a->stats.resident_bytes -= std::min(reclaimed, a->stats.resident_bytes);
        a->stats.resident_matrices = a->resident.size();
        ++a->stats.evicted;
        if (rc != VL_OK) return rc;
    }
    if (total > a->opt.maximum_resident_bytes - a->stats.resident_bytes) return VL_OK;
    vl_accel::Held h;
    // Out of budget or device memory is a reason to stop offering, not to fail the pass.
    if (acquire(a, VL_KIND_VRAM, total, "vl-accel-resident", &h) != VL_OK) return VL_OK;
    const auto t0 = std::chrono::steady_clock::now();
    int rc = a->be.upload(a->be.ctx, m.ggml_type, m.rows, m.storage_columns, m.encoded, h.ptr,
                          a->staging.ptr, a->scratch.ptr, a->opt.staging_bytes);
    a->stats.upload_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    if (rc != VL_OK) {
        const int rel = give_back(a, VL_KIND_VRAM, &h);
        return rel != VL_OK ? rel : rc;
    }
    vl_accel::Resident r;
    r.tiled = h.ptr;
    r.reservation = h.reservation;
    r.total_bytes = total;
    r.matrix_bytes = L.gguf_bytes;
    r.last_used = ++a->clock;
    r.rows = m.rows;
    r.cols = m.storage_columns;
    r.type = m.ggml_type;
    r.recurring = m.recurring != 0;
    try {
        it = a->resident.emplace(m.cache_identity, r).first;
    } catch (const std::bad_alloc&) {
        (void)give_back(a, VL_KIND_VRAM, &h);
        return fail(VL_RESOURCE_EXHAUSTED, "unable to record a resident matrix");
    }
    a->stats.uploaded_bytes += L.gguf_bytes;
    a->stats.resident_bytes += total;
    a->stats.resident_matrices = a->resident.size();
    *out = &it->second;
    return VL_OK;
}

// Grows the matvec I/O buffer to at least `bytes`; VL_RESOURCE_EXHAUSTED when refused.
int ensure_io(vl_accel* a, uint64_t bytes) {
    if (a->io.ptr && a->io.bytes >= bytes) return VL_OK;
    const int rc = give_back(a, VL_KIND_VRAM, &a->io);
    if (rc != VL_OK) return rc;
    return acquire(a, VL_KIND_VRAM, bytes, "vl-accel-io", &a->io);
}

}  // namespace

extern "C" {

void vl_accel_options_default(vl_accel_options* o) {
    if (!o) return;
    std::memset(o, 0, sizeof *o);
    o->device_ordinal = 0;
    o->experts_only = 0;
    o->minimum_free_vram_after = 1ull << 30;
    o->maximum_resident_bytes = 6ull << 30;
    o->maximum_matrices = 512;
    o->staging_bytes = 64ull << 20;
}

int vl_accel_create(const vl_accel_options* options, const vl_governor_ops* governor,
                    const vl_accel_backend* backend, vl_accel** out) {
    if (!options || !out) return fail(VL_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    if (!ops_valid(governor)) return fail(VL_INVALID_ARGUMENT, "a governor is required");
    if (options->device_ordinal < 0) return fail(VL_INVALID_ARGUMENT, "device ordinal cannot be negative");
    if (options->staging_bytes < 2u * 4096u) return fail(VL_INVALID_ARGUMENT, "staging_bytes is too small");
    if (backend && (!backend->free_memory || !backend->allocate || !backend->release ||
                    !backend->upload || !backend->io_bytes || !backend->matvec))
        return fail(VL_INVALID_ARGUMENT, "incomplete backend");
    vl_accel* a = new (std::nothrow) vl_accel;
    if (!a) return fail(VL_RESOURCE_EXHAUSTED, "unable to allocate the accelerator");
    a->opt = *options;
    a->gov = *governor;
    if (backend) {
        a->be = *backend;
    } else {
        int rc = VL_OK;
        a->hip = hip_backend_create(options->device_ordinal, &rc);
        if (!a->hip) {
            delete a;
            return rc;
        }
        a->be.ctx = a->hip;
        a->be.free_memory = hb_free_memory;
        a->be.allocate = hb_allocate;
        a->be.release = hb_release;
        a->be.upload = hb_upload;
        a->be.io_bytes = hb_io_bytes;
        a->be.matvec = hb_matvec;
    }
    // Two pinned staging slots and two device scratch slots of the same size.
    int rc = acquire(a, VL_KIND_STAGING, options->staging_bytes, "vl-accel-staging", &a->staging);
    if (rc == VL_OK) rc = acquire(a, VL_KIND_VRAM, options->staging_bytes, "vl-accel-scratch", &a->scratch);
    if (rc != VL_OK) {
        vl_accel_destroy(a);
        return rc;
    }
    *out = a;
    return VL_OK;
}

int vl_accel_destroy(vl_accel* a) {
    if (!a) return VL_OK;
    if (a->hip) hb_synchronize(a->hip);
    int rc = VL_OK;
    for (auto& kv : a->resident) {
        const int r = release_resident(a, kv.second);
        if (rc == VL_OK) rc = r;
    }
    a->resident.clear();
    for (vl_accel::Held* h : {&a->io, &a->scratch}) {
        const int r = give_back(a, VL_KIND_VRAM, h);
        if (rc == VL_OK) rc = r;
    }
    const int r = give_back(a, VL_KIND_STAGING, &a->staging);
    if (rc == VL_OK) rc = r;
    if (a->hip) hip_backend_destroy(a->hip);
    delete a;
    return rc;
}

int vl_accel_matvec(vl_accel* a, const vl_packed_matrix* m, const float* input, uint64_t input_len,
                    float* output, uint64_t output_len) {
    if (!a || !m) return fail(VL_INVALID_ARGUMENT, "null argument");
    ++a->stats.offered;
    if (!input || !output || input_len != m->storage_columns || output_len != m->rows) {
        ++a->stats.declined;
        return fail(VL_DECLINED, "input/output spans do not match the matrix");
    }
    vl_accel::Resident* r = nullptr;
    int rc = ensure_resident(a, *m, &r);
    if (rc != VL_OK) return rc;
    if (!r) {
        ++a->stats.declined;
        return fail(VL_DECLINED, "matrix declined");
    }
    uint64_t io_bytes = 0;
    rc = a->be.io_bytes(a->be.ctx, r->type, r->rows, r->cols, &io_bytes);
    if (rc != VL_OK) return rc;
    if (ensure_io(a, io_bytes) != VL_OK) {
        ++a->stats.declined;
        return fail(VL_DECLINED, "no device memory for the matvec buffers");
    }
    const auto t0 = std::chrono::steady_clock::now();
    rc = a->be.matvec(a->be.ctx, r->type, r->rows, r->cols, r->tiled, input, output, a->io.ptr, a->io.bytes);
    if (rc != VL_OK) return rc;
    a->stats.kernel_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    ++a->stats.accelerated;
    return VL_OK;
}

int vl_accel_prefetch(vl_accel* a, const vl_packed_matrix* m) {
    if (!a || !m) return fail(VL_INVALID_ARGUMENT, "null argument");
    vl_accel::Resident* r = nullptr;
    const int rc = ensure_resident(a, *m, &r);
    if (rc != VL_OK) return rc;
    return r ? VL_OK : fail(VL_DECLINED, "matrix declined");
}

int vl_accel_holds(const vl_accel* a, uint64_t identity) {
    return a && identity != 0 && a->resident.count(identity) ? 1 : 0;
}

int vl_accel_resident_matrix(const vl_accel* a, uint64_t identity, const void** tiled) {
    if (!a || !tiled) return fail(VL_INVALID_ARGUMENT, "null argument");
    auto it = a->resident.find(identity);
    if (identity == 0 || it == a->resident.end())
        return fail(VL_NOT_FOUND, "matrix %llu is not resident", (unsigned long long)identity);
    *tiled = it->second.tiled;
    return VL_OK;
}

int vl_accel_stats_get(const vl_accel* a, vl_accel_stats* out) {
    if (!a || !out) return fail(VL_INVALID_ARGUMENT, "null argument");
    *out = a->stats;
    return VL_OK;
}

}  // extern "C"
