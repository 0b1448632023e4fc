// Host side of the device boundary: the Safety Governor, Governor-reserved allocations and the
// matvec accelerator with device residency (include/vastloom_hip.h). Plain C++; the only device
// work is in the HIP backend at the end of this file, which calls the kernels of vl_kernels.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <list>
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
// Governor: the behaviour of safety::ResourceGovernor (src/safety/resource_governor.cpp:19-214),
// written as data. A reservation passes through an ordered table of admission rules; the first
// rule that objects decides the status. The safety state is the largest level any pressure
// signal raises (a budget's fill ratio, an availability floor), stepped through a hysteresis
// function that climbs at once and descends one level per run of calm samples.
// ------------------------------------------------------------------------------------------

namespace {

constexpr uint32_t kKinds = 4;
constexpr uint32_t kHostKinds[] = {VL_KIND_RAM, VL_KIND_STAGING, VL_KIND_SCRATCH};

uint64_t sat_add(uint64_t a, uint64_t b) { return a > UINT64_MAX - b ? UINT64_MAX : a + b; }
uint64_t sat_mul(uint64_t a, uint64_t b) { return b && a > UINT64_MAX / b ? UINT64_MAX : a * b; }

}  // namespace

struct vl_governor {
    vl_resource_limits limits{};
    mutable std::mutex mutex;
    uint64_t used[kKinds]{};  // bytes held per kind
    uint32_t level = VL_STATE_NORMAL;
    uint32_t calm_samples = 0;  // consecutive samples below the current level
    uint64_t next_id = 1;
    struct Grant {
        uint32_t kind;
        uint64_t bytes;
    };
    std::unordered_map<uint64_t, Grant> grants;

    uint64_t budget(uint32_t kind) const {
        const uint64_t b[kKinds] = {limits.ram_hard_limit, limits.vram_hard_limit,
                                    limits.staging_hard_limit, limits.scratch_hard_limit};
        return kind < kKinds ? b[kind] : 0;
    }
    // Host-side bytes held (RAM, staging, scratch), saturating.
    uint64_t host_used() const {
        uint64_t t = 0;
        for (uint32_t k : kHostKinds) t = sat_add(t, used[k]);
        return t;
    }
};

namespace {

const char* const kKindNames[kKinds] = {"ram", "vram", "staging", "scratch"};
const char* const kLevelNames[4] = {"normal", "pressure", "critical", "emergency"};

struct Request {
    uint32_t kind;
    uint64_t bytes;
    const char* tag;
};

// Admission rules, in the order they are consulted. Each returns VL_OK to let the request pass.
int admit_nonzero(const vl_governor&, const Request& r) {
    return r.bytes ? VL_OK : fail(VL_INVALID_ARGUMENT, "governor: empty request (%s)", r.tag);
}
int admit_open(const vl_governor& g, const Request& r) {
    return g.level < VL_STATE_CRITICAL
               ? VL_OK
               : fail(VL_RESOURCE_EXHAUSTED, "governor: closed to new work while %s (%s)",
                      kLevelNames[g.level], r.tag);
}
int admit_kind_budget(const vl_governor& g, const Request& r) {
    const uint64_t cap = g.budget(r.kind);
    const bool fits = cap != 0 && r.bytes <= cap && g.used[r.kind] <= cap - r.bytes;
    return fits ? VL_OK
                : fail(VL_RESOURCE_EXHAUSTED, "governor: %s budget cannot take %llu more bytes (%s)",
                       kKindNames[r.kind], (unsigned long long)r.bytes, r.tag);
}
int admit_host_total(const vl_governor& g, const Request& r) {
    const uint64_t cap = g.limits.host_memory_hard_limit;
    if (r.kind == VL_KIND_VRAM || cap == 0) return VL_OK;
    const uint64_t held = g.host_used();
    if (held > cap)
        return fail(VL_INTEGRITY_ERROR, "governor: host bytes held already exceed the host budget (%s)", r.tag);
    return r.bytes <= cap - held
               ? VL_OK
               : fail(VL_RESOURCE_EXHAUSTED, "governor: host budget cannot take %llu more bytes (%s)",
                      (unsigned long long)r.bytes, r.tag);
}
using AdmissionRule = int (*)(const vl_governor&, const Request&);
constexpr AdmissionRule kAdmission[] = {admit_nonzero, admit_open, admit_kind_budget, admit_host_total};

// Level signalled by a budget holding `held` of `cap` bytes (no signal without a budget).
uint32_t fill_level(uint64_t held, uint64_t cap, const vl_resource_limits& l) {
    if (cap == 0) return VL_STATE_NORMAL;
    const double ratio = (double)held / (double)cap;
    return ratio >= l.critical_ratio ? VL_STATE_CRITICAL
         : ratio >= l.pressure_ratio ? VL_STATE_PRESSURE
                                     : VL_STATE_NORMAL;
}

// Level signalled by `avail` bytes against a configured floor: a quarter of the floor or less is
// an emergency, the floor or less critical, twice the floor or less pressure.
uint32_t floor_level(uint64_t avail, uint64_t floor) {
    static constexpr struct {
        uint64_t num, den;
        uint32_t level;
    } kSteps[] = {{1, 4, VL_STATE_EMERGENCY}, {1, 1, VL_STATE_CRITICAL}, {2, 1, VL_STATE_PRESSURE}};
    for (const auto& st : kSteps)
        if (avail <= sat_mul(floor, st.num) / st.den) return st.level;
    return VL_STATE_NORMAL;
}

// One sample of the hysteresis: a higher level is taken at once; a lower one only after
// recovery_samples consecutive lower samples, and then one level at a time.
void settle(vl_governor& g, uint32_t signalled) {
    if (signalled > g.level) {
        g.level = signalled;
        g.calm_samples = 0;
    } else if (signalled == g.level) {
        g.calm_samples = 0;
    } else if (++g.calm_samples >= g.limits.recovery_samples) {
        --g.level;
        g.calm_samples = 0;
    }
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
    // The ratios are kept in [0.10, 0.99] and above the pressure ratio, and at least one calm
    // sample is needed to recover (ResourceGovernor::ResourceGovernor, resource_governor.cpp:58-62).
    vl_resource_limits& l = g->limits;
    l.pressure_ratio = std::clamp(l.pressure_ratio, 0.10, 0.99);
    l.critical_ratio = std::clamp(l.critical_ratio, l.pressure_ratio + 0.01, 1.0);
    l.recovery_samples = std::max(1u, l.recovery_samples);
    *out = g;
    return VL_OK;
}

void vl_governor_destroy(vl_governor* g) { delete g; }

int vl_governor_try_reserve(vl_governor* g, uint32_t kind, uint64_t bytes, const char* tag,
                            uint64_t* id) {
    if (!g || !id) return fail(VL_INVALID_ARGUMENT, "null argument");
    if (kind >= kKinds) return fail(VL_INVALID_ARGUMENT, "governor: unknown resource kind %u", kind);
    const Request req{kind, bytes, tag ? tag : ""};
    if (!bytes) return admit_nonzero(*g, req);
    std::lock_guard<std::mutex> lock(g->mutex);
    for (AdmissionRule rule : kAdmission)
        if (const int rc = rule(*g, req)) return rc;
    try {
        g->grants.emplace(g->next_id, vl_governor::Grant{kind, bytes});
    } catch (const std::bad_alloc&) {
        return fail(VL_RESOURCE_EXHAUSTED, "governor: no memory to record the grant (%s)", req.tag);
    }
    g->used[kind] += bytes;
    *id = g->next_id++;
    return VL_OK;
}

int vl_governor_release(vl_governor* g, uint64_t id) {
    if (!g) return fail(VL_INVALID_ARGUMENT, "null governor");
    std::lock_guard<std::mutex> lock(g->mutex);
    const auto it = g->grants.find(id);
    if (it == g->grants.end()) return fail(VL_NOT_FOUND, "governor: no grant %llu", (unsigned long long)id);
    uint64_t& u = g->used[it->second.kind];
    u -= std::min(u, it->second.bytes);
    g->grants.erase(it);
    return VL_OK;
}

int vl_governor_abandon(vl_governor* g, uint64_t id) {
    if (!g) return fail(VL_INVALID_ARGUMENT, "null governor");
    std::lock_guard<std::mutex> lock(g->mutex);
    // The grant is forgotten but its bytes stay in used[]: memory that could not be freed must not
    // be handed out again.
    if (!g->grants.erase(id)) return fail(VL_NOT_FOUND, "governor: no grant %llu", (unsigned long long)id);
    return VL_OK;
}

int vl_governor_update_pressure(vl_governor* g, const vl_runtime_pressure* p, uint32_t* state) {
    if (!g || !p) return fail(VL_INVALID_ARGUMENT, "null argument");
    std::lock_guard<std::mutex> lock(g->mutex);
    const vl_resource_limits& l = g->limits;
    uint32_t signals[kKinds + 3];
    uint32_t n = 0;
    for (uint32_t k = 0; k < kKinds; ++k) signals[n++] = fill_level(g->used[k], g->budget(k), l);
    signals[n++] = fill_level(std::min(g->host_used(), l.host_memory_hard_limit), l.host_memory_hard_limit, l);
    signals[n++] = floor_level(p->system_ram_available, l.minimum_system_ram_available);
    signals[n++] = floor_level(p->storage_available, l.minimum_storage_available);
    settle(*g, *std::max_element(signals, signals + n));
    if (state) *state = g->level;
    return VL_OK;
}

int vl_governor_snapshot_get(const vl_governor* g, vl_governor_snapshot* out) {
    if (!g || !out) return fail(VL_INVALID_ARGUMENT, "null argument");
    std::lock_guard<std::mutex> lock(g->mutex);
    out->state = g->level;
    out->recovery_counter = g->calm_samples;
    std::copy(g->used, g->used + kKinds, out->reserved);
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
    // The matrix is complete when the upload returns (as the reference's synchronous
    // copy_from_host leaves it): its pointer may be handed to kernels on any stream, and the
    // upload time covers the whole transfer.
    if (rc == VL_OK) rc = hip_check(hipStreamSynchronize(hb->compute), "hipStreamSynchronize");
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
// Accelerator: the residency policy of CudaMatvecAccelerator
// (src/cuda/cuda_matvec_accelerator.cpp:102-314). A matrix offered for the first time is
// classified (taken, or declined for one of the policy's reasons); a taken matrix that is not
// resident is uploaded after room is made. Resident matrices sit in two recency queues: the
// matrices whose descriptors say they will not be asked for again this pass, and the recurring
// ones. Room is made from the front (least recently used end) of the first queue, and only when
// it is empty from the second, so a pass's stream of routed experts cannot push out the weights
// every token needs. A hit moves a matrix to the back of its queue.
// ------------------------------------------------------------------------------------------

struct vl_accel {
    struct Held {  // a Governor-reserved device or pinned allocation
        void* ptr = nullptr;
        uint64_t reservation = 0;
        uint64_t bytes = 0;
    };
    struct Resident {
        Held mem;                  // tiled matrix (device)
        uint64_t rows = 0, cols = 0;
        uint32_t type = 0;
        bool recurring = false;
        std::list<uint64_t>::iterator queue_pos;  // in queue[recurring]
    };
    vl_accel_options opt{};
    vl_governor_ops gov{};
    vl_accel_backend be{};
    HipBackend* hip = nullptr;  // owned when be is the HIP backend
    std::unordered_map<uint64_t, Resident> resident;
    std::list<uint64_t> queue[2];  // [0] not recurring, [1] recurring; front = least recently used
    vl_accel_stats stats{};
    Held staging, scratch, io;
};

namespace {

// Every type with a device layout: the four tiled types and the GGUF-layout ones (Q4_K, Q5_K,
// Q6_K, IQ2_S, MXFP4, BF16, F32): the storage types the reference's accelerator takes
// (src/cuda/cuda_matvec_accelerator.cpp:46-58), and IQ2_S.
bool has_kernel(uint32_t type) {
    uint32_t elems = 0, bytes = 0;
    return vl_block_shape(type, &elems, &bytes) != 0;
}

// Counts a declined storage type in the first free or matching slot; types beyond the slots go
// uncounted (a statistic, never a failure).
void count_declined_type(vl_accel_stats& st, uint32_t type) {
    for (uint32_t i = 0; i < VL_ACCEL_TYPE_SLOTS; ++i) {
        if (st.declined_by_type[i] == 0) st.declined_type[i] = type;
        if (st.declined_type[i] == type) {
            ++st.declined_by_type[i];
            return;
        }
    }
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
    *h = vl_accel::Held{};
    return rc;
}

// Why an offered matrix is or is not taken.
enum class Offer { kTake, kRecurringRefused, kNoKernel, kBadShape, kNoIdentity };

Offer classify(const vl_accel& a, const vl_packed_matrix& m) {
    if (a.opt.experts_only && m.recurring) return Offer::kRecurringRefused;
    if (!has_kernel(m.ggml_type)) return Offer::kNoKernel;
    uint32_t elems = 0, bytes = 0;
    vl_block_shape(m.ggml_type, &elems, &bytes);
    if (!m.rows || !m.storage_columns || m.storage_columns % elems) return Offer::kBadShape;
    return m.cache_identity ? Offer::kTake : Offer::kNoIdentity;
}

// Drops one resident matrix: the front of the not-recurring queue, else of the recurring one.
int evict_one(vl_accel* a) {
    std::list<uint64_t>& q = a->queue[0].empty() ? a->queue[1] : a->queue[0];
    const auto it = a->resident.find(q.front());
    q.pop_front();
    const uint64_t freed = it->second.mem.bytes;
    const int rc = give_back(a, VL_KIND_VRAM, &it->second.mem);
    a->resident.erase(it);
    a->stats.resident_bytes -= std::min(freed, a->stats.resident_bytes);
    a->stats.resident_matrices = a->resident.size();
    ++a->stats.evicted;
    return rc;
}

// The resident entry for this matrix, uploading it on first sight; *out stays null when the
// accelerator declines it (a decline is not an error: the caller runs its CPU path).
int ensure_resident(vl_accel* a, const vl_packed_matrix& m, vl_accel::Resident** out) {
    *out = nullptr;
    switch (classify(*a, m)) {
        case Offer::kRecurringRefused: ++a->stats.declined_recurring; return VL_OK;
        case Offer::kNoKernel: count_declined_type(a->stats, m.ggml_type); return VL_OK;
        case Offer::kBadShape:
        case Offer::kNoIdentity: return VL_OK;
        case Offer::kTake: break;
    }
    if (const auto hit = a->resident.find(m.cache_identity); hit != a->resident.end()) {
        vl_accel::Resident& r = hit->second;
        auto& q = a->queue[r.recurring];
        q.splice(q.end(), q, r.queue_pos);
        *out = &r;
        return VL_OK;
    }
    if (!m.encoded) return fail(VL_INVALID_ARGUMENT, "matrix %llu has no payload", (unsigned long long)m.cache_identity);
    vl_tiled_layout L;
    const bool fits32 = m.rows <= 0x7fffffffu && m.storage_columns <= 0x7fffffffu;
    if (!fits32 || !vl_make_layout(m.ggml_type, (uint32_t)m.rows, (uint32_t)m.storage_columns, &L) ||
        m.encoded_bytes != L.gguf_bytes)
        return VL_OK;
    const uint64_t need = L.bytes, cap = a->opt.maximum_resident_bytes;
    if (need > cap) return VL_OK;
    auto crowded = [&] {
        return a->stats.resident_bytes + need > cap || a->resident.size() >= a->opt.maximum_matrices;
    };
    while (crowded() && !a->resident.empty())
        if (const int rc = evict_one(a)) return rc;
    if (need > cap - a->stats.resident_bytes) return VL_OK;
    vl_accel::Resident r;
    // A Governor or free-memory refusal declines the matrix; it does not fail the pass.
    if (acquire(a, VL_KIND_VRAM, need, "vl-accel-resident", &r.mem) != VL_OK) return VL_OK;
    const auto t0 = std::chrono::steady_clock::now();
    const int up = a->be.upload(a->be.ctx, m.ggml_type, m.rows, m.storage_columns, m.encoded, r.mem.ptr,
                                a->staging.ptr, a->scratch.ptr, a->opt.staging_bytes);
    a->stats.upload_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    if (up != VL_OK) {
        const int rel = give_back(a, VL_KIND_VRAM, &r.mem);
        return rel != VL_OK ? rel : up;
    }
    r.rows = m.rows;
    r.cols = m.storage_columns;
    r.type = m.ggml_type;
    r.recurring = m.recurring != 0;
    try {
        auto& q = a->queue[r.recurring];
        q.push_back(m.cache_identity);
        r.queue_pos = std::prev(q.end());
        try {
            *out = &a->resident.emplace(m.cache_identity, r).first->second;
        } catch (...) {
            q.pop_back();
            throw;
        }
    } catch (const std::bad_alloc&) {
        (void)give_back(a, VL_KIND_VRAM, &r.mem);
        return fail(VL_RESOURCE_EXHAUSTED, "unable to record a resident matrix");
    }
    a->stats.uploaded_bytes += L.gguf_bytes;
    a->stats.resident_bytes += need;
    a->stats.resident_matrices = a->resident.size();
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
        const int r = give_back(a, VL_KIND_VRAM, &kv.second.mem);
        if (rc == VL_OK) rc = r;
    }
    a->resident.clear();
    a->queue[0].clear();
    a->queue[1].clear();
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
    rc = a->be.matvec(a->be.ctx, r->type, r->rows, r->cols, r->mem.ptr, input, output, a->io.ptr, a->io.bytes);
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
    *tiled = it->second.mem.ptr;
    return VL_OK;
}

int vl_accel_stats_get(const vl_accel* a, vl_accel_stats* out) {
    if (!a || !out) return fail(VL_INVALID_ARGUMENT, "null argument");
    *out = a->stats;
    return VL_OK;
}

}  // extern "C"
