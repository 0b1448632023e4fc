// C ABI entry points (include/vastloom_hip.h) over the HIP kernels.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "../../include/vastloom_hip.h"
#include "vl_error.h"
#include "vl_kernels.h"
#include "vl_layout.h"
#include "vl_moe.h"

namespace {
thread_local std::string g_last_error;
}  // namespace

int vl::fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

namespace {

using vl::fail;

int hip_fail(hipError_t e, const char* what) {
    return fail(VL_INTERNAL_ERROR, "%s: %s", what, hipGetErrorString(e));
}

bool make_layout(uint32_t type, uint64_t rows, uint64_t cols, vl_tiled_layout* L) {
    if (rows == 0 || cols == 0 || rows > 0x7fffffffu || cols > 0x7fffffffu) return false;
    return vl_make_layout(type, (uint32_t)rows, (uint32_t)cols, L) != 0;
}

// The status word sits at the start of every workspace.
constexpr uint64_t kStatusOffset = 0;

// Persistent blocks of the current device, or 0 with the error recorded.
uint32_t blocks_or_fail() {
    const uint32_t b = vl::stream_blocks();
    if (b == 0) fail(VL_UNSUPPORTED, "no HIP device is current");
    return b;
}

}  // namespace

extern "C" {

const char* vl_last_error(void) { return g_last_error.c_str(); }

int vl_device_count(int* count) {
    if (!count) return fail(VL_INVALID_ARGUMENT, "count is null");
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) n = 0;
    else if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    *count = n;
    return VL_OK;
}

int vl_gpu_probe(int device, vl_gpu_info* out) {
    if (!out) return fail(VL_INVALID_ARGUMENT, "out is null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess && e != hipErrorNoDevice) return hip_fail(e, "hipGetDeviceCount");
    if (e == hipErrorNoDevice || device < 0 || device >= n)
        return fail(VL_INVALID_ARGUMENT, "no HIP device %d", device);
    hipDeviceProp_t prop{};
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    int cur = 0;
    if ((e = hipGetDevice(&cur)) != hipSuccess) return hip_fail(e, "hipGetDevice");
    if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    size_t free_b = 0, total_b = 0;
    e = hipMemGetInfo(&free_b, &total_b);
    (void)hipSetDevice(cur);
    if (e != hipSuccess) return hip_fail(e, "hipMemGetInfo");
    int drv = 0;
    if ((e = hipDriverGetVersion(&drv)) != hipSuccess) return hip_fail(e, "hipDriverGetVersion");
    vl_gpu_info g{};
    std::snprintf(g.backend, sizeof g.backend, "%s", "hip");
    std::snprintf(g.name, sizeof g.name, "%s", prop.name);
    std::snprintf(g.arch, sizeof g.arch, "%s", prop.gcnArchName);
    std::snprintf(g.driver_version, sizeof g.driver_version, "%d", drv);
    g.total_vram_bytes = total_b;
    g.free_vram_bytes = free_b;
    g.compute_units = (uint32_t)prop.multiProcessorCount;
    *out = g;
    return VL_OK;
}

int vl_matrix_layout(uint32_t type, uint64_t rows, uint64_t cols, uint64_t* gguf_bytes,
                     uint64_t* device_bytes) {
    vl_tiled_layout L;
    if (!make_layout(type, rows, cols, &L))
        return fail(VL_UNSUPPORTED, "no device layout for type %u with %llu x %llu", type,
                    (unsigned long long)rows, (unsigned long long)cols);
    if (gguf_bytes) *gguf_bytes = L.gguf_bytes;
    if (device_bytes) *device_bytes = L.bytes;
    return VL_OK;
}

int vl_pack_matrix(uint32_t type, uint64_t rows, uint64_t cols, const void* gguf_device,
                   void* tiled_device, void* stream) {
    vl_tiled_layout L;
    if (!make_layout(type, rows, cols, &L)) return fail(VL_UNSUPPORTED, "unsupported matrix");
    if (!gguf_device || !tiled_device) return fail(VL_INVALID_ARGUMENT, "null device pointer");
    const hipError_t e = vl::launch_pack(L, static_cast<const uint8_t*>(gguf_device),
                                         static_cast<uint8_t*>(tiled_device),
                                         static_cast<hipStream_t>(stream));
    return e == hipSuccess ? VL_OK : hip_fail(e, "pack launch");
}

int vl_dequantize(uint32_t type, uint64_t rows, uint64_t cols, const void* tiled_device,
                  float* out_device, void* stream) {
    vl_tiled_layout L;
    if (!make_layout(type, rows, cols, &L)) return fail(VL_UNSUPPORTED, "unsupported matrix");
    if (!tiled_device || !out_device) return fail(VL_INVALID_ARGUMENT, "null device pointer");
    const hipError_t e = vl::launch_dequant(L, static_cast<const uint8_t*>(tiled_device),
                                            out_device, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? VL_OK : hip_fail(e, "dequantize launch");
}

int vl_matvec_workspace(uint32_t type, uint64_t rows, uint64_t cols, uint32_t tokens,
                        uint64_t* bytes) {
    vl_tiled_layout L;
    if (!make_layout(type, rows, cols, &L)) return fail(VL_UNSUPPORTED, "unsupported matrix");
    if (tokens == 0 || tokens > 8) return fail(VL_INVALID_ARGUMENT, "tokens must be 1..8");
    if (!bytes) return fail(VL_INVALID_ARGUMENT, "bytes is null");
    const uint32_t blocks = blocks_or_fail();
    if (!blocks) return VL_UNSUPPORTED;
    *bytes = vl::matvec_workspace_bytes(type, (uint32_t)rows, (uint32_t)cols, tokens, blocks);
    return VL_OK;
}

int vl_matvec(uint32_t type, uint64_t rows, uint64_t cols, const void* tiled_device,
              const float* x_device, uint32_t tokens, float* y_device, void* workspace,
              uint64_t workspace_bytes, void* stream) {
    uint64_t need = 0;
    int st = vl_matvec_workspace(type, rows, cols, tokens, &need);
    if (st) return st;
    if (!tiled_device || !x_device || !y_device || !workspace)
        return fail(VL_INVALID_ARGUMENT, "null device pointer");
    if (workspace_bytes < need)
        return fail(VL_INVALID_ARGUMENT, "workspace of %llu bytes is below the %llu needed",
                    (unsigned long long)workspace_bytes, (unsigned long long)need);
    vl_tiled_layout L;
    make_layout(type, rows, cols, &L);
    const hipError_t e = vl::launch_matvec(L, static_cast<const uint8_t*>(tiled_device), x_device,
                                           tokens, y_device, static_cast<uint8_t*>(workspace),
                                           vl::stream_blocks(), static_cast<hipStream_t>(stream));
    return e == hipSuccess ? VL_OK : hip_fail(e, "matvec launch");
}

static bool to_shape(const vl_moe_config* c, vl::MoeShape* s) {
    if (!c) return false;
    *s = vl::MoeShape{c->tokens, c->width, c->intermediate, c->experts, c->top_k,
                      c->gate_type, c->down_type, c->semantics, c->routing, c->score_fn,
                      c->has_shared, c->renormalize, c->route_scale, c->routed_limit,
                      c->shared_limit};
    return vl::moe_shape_ok(*s);
}

int vl_moe_workspace(const vl_moe_config* config, uint64_t* bytes) {
    vl::MoeShape s;
    if (!to_shape(config, &s)) return fail(VL_INVALID_ARGUMENT, "invalid MoE configuration");
    if (!bytes) return fail(VL_INVALID_ARGUMENT, "bytes is null");
    const uint32_t blocks = blocks_or_fail();
    if (!blocks) return VL_UNSUPPORTED;
    *bytes = vl::moe_workspace_bytes(s, blocks);
    return VL_OK;
}

// Everything a layer call checks before it launches: the configuration, the pointers its routing
// and semantics read, and the workspace size. Fills the launch arguments on success.
static int prepare_moe(const vl_moe_config* config, const vl_moe_inputs* inputs, void* workspace,
                       uint64_t workspace_bytes, vl::MoeShape* s, vl::MoeInputs* in,
                       vl::MoeWorkspace* ws) {
    if (!to_shape(config, s)) return fail(VL_INVALID_ARGUMENT, "invalid MoE configuration");
    if (!inputs || !inputs->experts || !inputs->x || !inputs->out || !workspace)
        return fail(VL_INVALID_ARGUMENT, "null input pointer");
    if (s->routing != vl::kRouteGiven && !inputs->router)
        return fail(VL_INVALID_ARGUMENT, "routing needs the router weights");
    if (s->routing == vl::kRouteTable && !inputs->table_ids)
        return fail(VL_INVALID_ARGUMENT, "table routing needs table ids");
    const uint32_t blocks = blocks_or_fail();
    if (!blocks) return VL_UNSUPPORTED;
    *ws = vl::moe_workspace_layout(*s, blocks, workspace);
    if (workspace_bytes < ws->bytes)
        return fail(VL_INVALID_ARGUMENT, "workspace of %llu bytes is below the %llu needed",
                    (unsigned long long)workspace_bytes, (unsigned long long)ws->bytes);
    *in = vl::MoeInputs{reinterpret_cast<const vl::MoeExpert*>(inputs->experts), inputs->router,
                        inputs->bias, inputs->table_ids, inputs->given_ids, inputs->given_weights,
                        inputs->x, inputs->out};
    return VL_OK;
}

int vl_moe_layer(const vl_moe_config* config, const vl_moe_inputs* inputs, void* workspace,
                 uint64_t workspace_bytes, void* stream) {
    vl::MoeShape s;
    vl::MoeInputs in;
    vl::MoeWorkspace ws;
    if (const int rc = prepare_moe(config, inputs, workspace, workspace_bytes, &s, &in, &ws)) return rc;
    const hipError_t e = vl::launch_moe(s, in, ws, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? VL_OK : hip_fail(e, "MoE launch");
}

int vl_moe_route(const vl_moe_config* config, const vl_moe_inputs* inputs, void* workspace,
                 uint64_t workspace_bytes, void* stream) {
    vl::MoeShape s;
    if (!to_shape(config, &s)) return fail(VL_INVALID_ARGUMENT, "invalid MoE configuration");
    if (s.routing == vl::kRouteGiven) return fail(VL_INVALID_ARGUMENT, "given routes need no routing");
    if (!inputs || !inputs->router || !inputs->x || !workspace)
        return fail(VL_INVALID_ARGUMENT, "null input pointer");
    if (s.routing == vl::kRouteTable && !inputs->table_ids)
        return fail(VL_INVALID_ARGUMENT, "table routing needs table ids");
    const uint32_t blocks = blocks_or_fail();
    if (!blocks) return VL_UNSUPPORTED;
    const vl::MoeWorkspace ws = vl::moe_workspace_layout(s, blocks, workspace);
    if (workspace_bytes < ws.bytes)
        return fail(VL_INVALID_ARGUMENT, "workspace of %llu bytes is below the %llu needed",
                    (unsigned long long)workspace_bytes, (unsigned long long)ws.bytes);
    // The experts are not read: the table pointer is only carried.
    const vl::MoeInputs in{reinterpret_cast<const vl::MoeExpert*>(inputs->experts), inputs->router, inputs->bias,
                           inputs->table_ids, nullptr, nullptr, inputs->x, inputs->out};
    const hipError_t e = vl::launch_moe_route(s, in, ws, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? VL_OK : hip_fail(e, "MoE routing launch");
}

int vl_moe_layer_noalloc(const vl_moe_config* config, const vl_moe_inputs* inputs, void* stream) {
    vl::MoeShape s;
    if (!to_shape(config, &s)) return fail(VL_INVALID_ARGUMENT, "invalid MoE configuration");
    const uint32_t blocks = blocks_or_fail();
    if (!blocks) return VL_UNSUPPORTED;
    const uint64_t need = vl::moe_workspace_bytes(s, blocks);
    if (need > vl::kStaticWorkspaceBytes)
        return fail(VL_RESOURCE_EXHAUSTED,
                    "this layer needs a %llu-byte workspace; the static workspace holds %llu bytes "
                    "(use vl_moe_layer with a caller-owned workspace)",
                    (unsigned long long)need, (unsigned long long)vl::kStaticWorkspaceBytes);
    void* ws_ptr = nullptr;
    const hipError_t se = vl::static_workspace(&ws_ptr);
    if (se != hipSuccess) return hip_fail(se, "static workspace lookup");
    vl::MoeInputs in;
    vl::MoeWorkspace ws;
    if (const int rc = prepare_moe(config, inputs, ws_ptr, vl::kStaticWorkspaceBytes, &s, &in, &ws)) return rc;
    const hipError_t e = vl::launch_moe(s, in, ws, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? VL_OK : hip_fail(e, "MoE launch");
}

int vl_moe_noalloc_status(void* stream, uint32_t* bits) {
    if (!bits) return fail(VL_INVALID_ARGUMENT, "bits is null");
    void* ws_ptr = nullptr;
    const hipError_t se = vl::static_workspace(&ws_ptr);
    if (se != hipSuccess) return hip_fail(se, "static workspace lookup");
    return vl_read_status(ws_ptr, stream, bits);
}

}  // extern "C"

struct vl_timeline {
    uint32_t calls = 0;
    bool brackets = false;                // record kernel brackets instead of stage marks
    std::vector<hipEvent_t> events;       // calls x (stages + 1): marks between the stages
    std::vector<hipEvent_t> kernels;      // calls x 2 stages: start and stop of each stage's kernel
    std::vector<uint8_t> bracketed;       // per call: kernels recorded
};

extern "C" {

int vl_timeline_create(uint32_t calls, vl_timeline** out) {
    if (!out || calls == 0) return fail(VL_INVALID_ARGUMENT, "invalid timeline request");
    auto* t = new (std::nothrow) vl_timeline;
    if (!t) return fail(VL_RESOURCE_EXHAUSTED, "timeline allocation failed");
    t->calls = calls;
    t->events.assign((size_t)calls * (vl::kStageCount + 1), nullptr);
    t->kernels.assign((size_t)calls * 2u * vl::kStageCount, nullptr);
    t->bracketed.assign(calls, 0);
    for (auto* v : {&t->events, &t->kernels})
        for (auto& e : *v) {
            const hipError_t r = hipEventCreate(&e);
            if (r != hipSuccess) {
                vl_timeline_destroy(t);
                return hip_fail(r, "hipEventCreate");
            }
        }
    *out = t;
    return VL_OK;
}

void vl_timeline_destroy(vl_timeline* t) {
    if (!t) return;
    for (auto* v : {&t->events, &t->kernels})
        for (auto e : *v)
            if (e) (void)hipEventDestroy(e);
    delete t;
}

int vl_timeline_set_kernel_brackets(vl_timeline* t, int enabled) {
    if (!t) return fail(VL_INVALID_ARGUMENT, "timeline is null");
    t->brackets = enabled != 0;
    return VL_OK;
}

int vl_moe_layer_profiled(const vl_moe_config* config, const vl_moe_inputs* inputs,
                          void* workspace, uint64_t workspace_bytes, void* stream,
                          vl_timeline* timeline, uint32_t call) {
    vl::MoeShape s;
    vl::MoeInputs in;
    vl::MoeWorkspace ws;
    if (const int rc = prepare_moe(config, inputs, workspace, workspace_bytes, &s, &in, &ws)) return rc;
    if (!timeline || call >= timeline->calls) return fail(VL_INVALID_ARGUMENT, "bad timeline slot");
    hipEvent_t* ev = timeline->events.data() + (size_t)call * (vl::kStageCount + 1);
    hipEvent_t* kev = timeline->kernels.data() + (size_t)call * 2u * vl::kStageCount;
    timeline->bracketed[call] = timeline->brackets ? 1 : 0;
    const hipError_t e = vl::launch_moe(s, in, ws, static_cast<hipStream_t>(stream),
                                        timeline->brackets ? nullptr : ev,
                                        timeline->brackets ? kev : nullptr);
    return e == hipSuccess ? VL_OK : hip_fail(e, "MoE launch");
}

int vl_timeline_stage_ms(vl_timeline* t, uint32_t call, float* ms) {
    if (!t || call >= t->calls || !ms) return fail(VL_INVALID_ARGUMENT, "bad timeline read");
    if (t->bracketed[call]) return fail(VL_INVALID_ARGUMENT, "call %u recorded kernel brackets", call);
    hipEvent_t* ev = t->events.data() + (size_t)call * (vl::kStageCount + 1);
    for (uint32_t i = 0; i < vl::kStageCount; ++i) {
        const hipError_t r = hipEventElapsedTime(&ms[i], ev[i], ev[i + 1]);
        if (r != hipSuccess) return hip_fail(r, "hipEventElapsedTime");
    }
    return VL_OK;
}

int vl_timeline_kernel_ms(vl_timeline* t, uint32_t call, float* ms) {
    if (!t || call >= t->calls || !ms) return fail(VL_INVALID_ARGUMENT, "bad timeline read");
    if (!t->bracketed[call]) return fail(VL_INVALID_ARGUMENT, "call %u recorded stage marks", call);
    hipEvent_t* ev = t->kernels.data() + (size_t)call * 2u * vl::kStageCount;
    for (uint32_t i = 0; i < vl::kStageCount; ++i) {
        const hipError_t r = hipEventElapsedTime(&ms[i], ev[2 * i], ev[2 * i + 1]);
        if (r != hipSuccess) return hip_fail(r, "hipEventElapsedTime");
    }
    return VL_OK;
}

int vl_moe_read_routes(const vl_moe_config* config, const void* workspace, void* stream,
                       uint32_t* ids_host, float* weights_host) {
    vl::MoeShape s;
    if (!to_shape(config, &s)) return fail(VL_INVALID_ARGUMENT, "invalid MoE configuration");
    if (!workspace || !ids_host || !weights_host) return fail(VL_INVALID_ARGUMENT, "null pointer");
    const uint32_t blocks = blocks_or_fail();
    if (!blocks) return VL_UNSUPPORTED;
    const vl::MoeWorkspace ws = vl::moe_workspace_layout(s, blocks, const_cast<void*>(workspace));
    const uint64_t n = (uint64_t)s.tokens * s.top_k;
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    if (e == hipSuccess)
        e = hipMemcpy(ids_host, ws.base + ws.off_route_idx, n * 4u, hipMemcpyDeviceToHost);
    if (e == hipSuccess)
        e = hipMemcpy(weights_host, ws.base + ws.off_route_w, n * 4u, hipMemcpyDeviceToHost);
    return e == hipSuccess ? VL_OK : hip_fail(e, "route read");
}

int vl_read_status(const void* workspace, void* stream, uint32_t* bits) {
    if (!workspace || !bits) return fail(VL_INVALID_ARGUMENT, "null pointer");
    const auto s = static_cast<hipStream_t>(stream);
    hipError_t e = hipStreamSynchronize(s);
    if (e == hipSuccess)
        e = hipMemcpy(bits, static_cast<const uint8_t*>(workspace) + kStatusOffset, sizeof(uint32_t),
                      hipMemcpyDeviceToHost);
    return e == hipSuccess ? VL_OK : hip_fail(e, "status read");
}

}  // extern "C"
