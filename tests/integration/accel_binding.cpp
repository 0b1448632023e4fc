// Drives integration/hip_matvec_accelerator.hpp, the reference-side binding, as the reference's
// graph would: through inference::DeepseekV4MatvecAccelerator::matvec, with the reference's own
// ResourceGovernor, DeepseekV4PackedMatrix and deepseek_v4_packed_matrix_payload, and the
// reference's CPU matvec (matvec_ggml_f32_transactional) as the expected result. Test
// infrastructure, built by `make -C oracle binding` into oracle/_ref/accel_binding.
//
//   accel_binding fake   device operations of host memory whose matvec is the reference's CPU
//                        kernel: outputs must be bit-identical to it (no GPU needed)
//   accel_binding hip    the HIP device: outputs within 1e-5 * |w_row| * |x| of the reference
//
// Each case prints "ok <name>" or "FAIL <name>: <why>"; the exit status is 1 if any failed. The
// cases follow the reference's own accelerator test (tests/test_cuda_driver.cpp:713-790): Ok(true)
// with the output written, Ok(false) with the output untouched (no identity, recurring weights under
// experts_only, a type without a kernel, too little budget), errors (a non-finite input, a failed
// upload), and the Governor's accounting through safety::Reservation.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "hip_matvec_accelerator.hpp"
#include "vastloom/inference/ggml_quantization.hpp"

namespace {

using namespace vastloom;
using inference::DeepseekV4PackedMatrix;

constexpr std::uint64_t MiB = 1ULL << 20;
int failures = 0;

void check(bool ok, const char* name, const std::string& why = {}) {
    if (ok) {
        std::printf("ok %s\n", name);
    } else {
        std::printf("FAIL %s: %s\n", name, why.c_str());
        ++failures;
    }
    std::fflush(stdout);
}

// splitmix64: the driver's own seeded byte source.
struct Rng {
    std::uint64_t s;
    std::uint64_t next() {
        std::uint64_t z = (s += 0x9e3779b97f4a7c15ULL);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
        return z ^ (z >> 31);
    }
    float normal() {  // Box-Muller on two uniform doubles
        const double u1 = ((next() >> 11) + 1.0) * 0x1.0p-53, u2 = (next() >> 11) * 0x1.0p-53;
        return static_cast<float>(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
};

// GGUF blocks with small finite fp16 scales: Q8_0 (34 B per 32 weights, quants in [-127, 127]) or
// IQ2_XXS (66 B per 256 weights, every payload byte valid).
std::vector<std::byte> random_blocks(std::uint32_t type, std::size_t rows, std::size_t cols, Rng& rng) {
    const bool q8 = type == inference::kGgmlTypeQ8_0;
    const std::size_t be = q8 ? 32 : 256, bb = q8 ? 34 : 66, blocks = rows * (cols / be);
    std::vector<std::byte> out(blocks * bb);
    for (std::size_t b = 0; b < blocks; ++b) {
        std::byte* p = out.data() + b * bb;
        const std::uint16_t d = static_cast<std::uint16_t>(0x1c00 + rng.next() % 0x0800);  // ~0.004 .. 0.016
        p[0] = static_cast<std::byte>(d & 0xff);
        p[1] = static_cast<std::byte>(d >> 8);
        for (std::size_t i = 2; i < bb; ++i) {
            const std::uint64_t r = rng.next();
            p[i] = q8 ? static_cast<std::byte>(static_cast<std::int8_t>(static_cast<int>(r % 255) - 127))
                      : static_cast<std::byte>(r & 0xff);
        }
    }
    return out;
}

DeepseekV4PackedMatrix matrix(std::uint32_t type, std::size_t rows, std::size_t cols, std::vector<std::byte> bytes,
                              std::uint64_t identity, bool recurring = false) {
    DeepseekV4PackedMatrix m(type, rows, cols, cols, std::move(bytes));
    m.cache_identity = identity;
    m.recurring = recurring;
    return m;
}

std::vector<float> reference_matvec(const DeepseekV4PackedMatrix& m, const std::vector<float>& x) {
    std::vector<float> scratch(m.rows), y(m.rows);
    auto r = inference::matvec_ggml_f32_transactional(m.ggml_type, m.encoded, m.rows, m.logical_columns, x, scratch, y);
    if (!r) std::printf("reference matvec failed: %s\n", r.error().message.c_str());
    return y;
}

// ---- Fake device: host memory, the reference's CPU matvec ------------------------------------

struct Fake {
    std::uint64_t free_bytes{1ULL << 40};
    std::map<void*, std::vector<std::byte>> mem;
    std::map<void*, DeepseekV4PackedMatrix> uploaded;
    bool fail_upload{false};
    int uploads{0}, matvecs{0};

    static Fake& of(void* c) { return *static_cast<Fake*>(c); }
    static int free_memory(void* c, int, std::uint64_t* out) {
        *out = of(c).free_bytes;
        return VL_OK;
    }
    static int allocate(void* c, std::uint32_t kind, int, std::uint64_t bytes, void** out) {
        Fake& f = of(c);
        std::vector<std::byte> buf(bytes ? bytes : 1);
        void* p = buf.data();
        f.mem.emplace(p, std::move(buf));
        if (kind == VL_KIND_VRAM) f.free_bytes -= bytes;
        *out = p;
        return VL_OK;
    }
    static int release(void* c, std::uint32_t kind, void* p) {
        Fake& f = of(c);
        auto it = f.mem.find(p);
        if (it != f.mem.end()) {
            if (kind == VL_KIND_VRAM) f.free_bytes += it->second.size();
            f.mem.erase(it);
        }
        f.uploaded.erase(p);
        return VL_OK;
    }
    static int upload(void* c, std::uint32_t type, std::uint64_t rows, std::uint64_t cols, const void* gguf,
                      void* tiled, void*, void*, std::uint64_t) {
        Fake& f = of(c);
        ++f.uploads;
        if (f.fail_upload) return 1 + static_cast<int>(ErrorCode::io_error);
        auto bytes = inference::ggml_storage_bytes(type, rows, cols);
        if (!bytes) return 1 + static_cast<int>(bytes.error().code);
        const auto* src = static_cast<const std::byte*>(gguf);
        f.uploaded.insert_or_assign(tiled, matrix(type, rows, cols, std::vector<std::byte>(src, src + bytes.value()), 0));
        return VL_OK;
    }
    static int io_bytes(void*, std::uint32_t, std::uint64_t rows, std::uint64_t cols, std::uint64_t* out) {
        *out = 4 * (rows + cols) + 256;
        return VL_OK;
    }
    static int matvec(void* c, std::uint32_t, std::uint64_t rows, std::uint64_t cols, const void* tiled, const float* x,
                      float* y, void*, std::uint64_t) {
        Fake& f = of(c);
        ++f.matvecs;
        auto it = f.uploaded.find(const_cast<void*>(tiled));
        if (it == f.uploaded.end()) return 1 + static_cast<int>(ErrorCode::internal_error);
        std::vector<float> scratch(rows);
        auto r = inference::matvec_ggml_f32_transactional(it->second.ggml_type, it->second.encoded, rows, cols,
                                                            std::span<const float>(x, cols), scratch,
                                                            std::span<float>(y, rows));
        return r ? VL_OK : 1 + static_cast<int>(r.error().code);
    }
    vl_accel_backend table() {
        return vl_accel_backend{this, &free_memory, &allocate, &release, &upload, &io_bytes, &matvec};
    }
};

safety::ResourceLimits limits(std::uint64_t vram, std::uint64_t staging) {
    safety::ResourceLimits l;
    l.ram_hard_limit = 256 * MiB;
    l.vram_hard_limit = vram;
    l.staging_hard_limit = staging;
    l.scratch_hard_limit = 64 * MiB;
    return l;
}

vl_accel_options options(std::uint64_t staging_bytes) {
    vl_accel_options o{};
    vl_accel_options_default(&o);
    o.staging_bytes = staging_bytes;
    o.minimum_free_vram_after = 0;
    return o;
}

bool untouched(const std::vector<float>& y) {
    for (float v : y)
        if (std::memcmp(&v, "\xef\xbe\xad\xde", 4) != 0) return false;
    return true;
}
std::vector<float> sentinel(std::size_t n) {
    std::vector<float> y(n);
    for (float& v : y) std::memcpy(&v, "\xef\xbe\xad\xde", 4);
    return y;
}

// Max over rows of |y - want| / (|w_row| * |x|), rows dequantized with the reference's decoder.
double worst_ratio(const DeepseekV4PackedMatrix& m, const std::vector<float>& x, const std::vector<float>& y,
                   const std::vector<float>& want) {
    double xn = 0.0;
    for (float v : x) xn += static_cast<double>(v) * v;
    xn = std::sqrt(xn);
    std::vector<float> row(m.logical_columns);
    double worst = 0.0;
    for (std::size_t r = 0; r < m.rows; ++r) {
        auto d = inference::dequantize_ggml_row_f32(m.ggml_type, m.encoded, m.rows, m.logical_columns, r, row);
        if (!d) return 1e30;
        double wn = 0.0;
        for (float v : row) wn += static_cast<double>(v) * v;
        const double err = std::fabs(static_cast<double>(y[r]) - want[r]);
        worst = std::max(worst, err / (std::sqrt(wn) * xn));
    }
    return worst;
}

std::uint64_t reserved(const safety::ResourceGovernor& g, safety::ResourceKind k) {
    return g.snapshot().reserved[static_cast<std::size_t>(k)];
}

int run(bool fake_device) {
    Fake fake;
    const vl_accel_backend table = fake.table();
    const vl_accel_backend* backend = fake_device ? &table : nullptr;
    const char* mode = fake_device ? "fake" : "hip";
    Rng rng{fake_device ? 11ULL : 12ULL};
    const std::uint32_t type = fake_device ? inference::kGgmlTypeQ8_0 : inference::kGgmlTypeIq2Xxs;
    const std::size_t rows = fake_device ? 96 : 512, cols = fake_device ? 512 : 2048;
    std::vector<float> x(cols);
    for (float& v : x) v = rng.normal();

    {
        safety::ResourceGovernor g(limits(64 * MiB, 16 * MiB));
        auto created = vastloom::hip::HipMatvecAccelerator::create(g, options(2 * MiB), backend);
        check(created.ok(), "create", created.ok() ? "" : created.error().message);
        if (!created) return 1;
        auto acc = created.take_value();
        // Two pinned staging slots and two device scratch slots, staging_bytes each in all.
        check(reserved(g, safety::ResourceKind::staging) == 2 * MiB && reserved(g, safety::ResourceKind::vram) == 2 * MiB &&
                  acc->reservations() == 2,
              "staging and scratch reserved through the reference Governor");

        // Ok(true): the output is the reference's (bit-identical on the fake device).
        auto m = matrix(type, rows, cols, random_blocks(type, rows, cols, rng), 0x51);
        auto y = sentinel(rows);
        auto r = acc->matvec(m, x, y);
        check(r.ok() && r.value(), "accelerated", r.ok() ? "declined" : r.error().message);
        const auto want = reference_matvec(m, x);
        if (fake_device) {
            check(std::memcmp(y.data(), want.data(), rows * 4) == 0, "fake output bit-identical to the reference");
        } else {
            const double w = worst_ratio(m, x, y, want);
            char why[64];
            std::snprintf(why, sizeof why, "max ratio %.3e", w);
            check(w <= 1e-5, "device output within 1e-5 |w_row| |x| of the reference", why);
        }
        check(acc->holds(0x51), "resident after first use");
        const std::uint64_t vram_now = reserved(g, safety::ResourceKind::vram);
        check(vram_now > 2 * MiB && acc->reservations() >= 3, "resident matrix reserved through the reference Governor");

        // Second use: no new upload, same output.
        const int uploads = fake.uploads;
        auto y2 = sentinel(rows);
        auto r2 = acc->matvec(m, x, y2);
        check(r2.ok() && r2.value() && std::memcmp(y2.data(), y.data(), rows * 4) == 0 &&
                  (!fake_device || fake.uploads == uploads),
              "second use reuses the resident copy");

        // Ok(false), output untouched: no identity; a type without a kernel.
        auto anon = matrix(type, rows, cols, m.encoded, 0);
        auto y3 = sentinel(rows);
        auto r3 = acc->matvec(anon, x, y3);
        check(r3.ok() && !r3.value() && untouched(y3), "no identity declined, output untouched");
        std::vector<std::byte> i32(rows * cols * 4);  // I32 storage has no device kernel
        auto q4 = matrix(inference::kGgmlTypeI32, rows, cols, i32, 0x52);
        auto y4 = sentinel(rows);
        auto r4 = acc->matvec(q4, x, y4);
        check(r4.ok() && !r4.value() && untouched(y4), "type without a kernel declined, output untouched");

        // An error, output untouched: a non-finite input.
        auto xbad = x;
        xbad[3] = NAN;
        auto y5 = sentinel(rows);
        auto r5 = acc->matvec(m, xbad, y5);
        check(!r5.ok() && r5.error().code == ErrorCode::invalid_argument && untouched(y5),
              "non-finite input is an error, output untouched",
              r5.ok() ? "not an error" : r5.error().message);

        auto st = acc->stats();
        check(st.ok() && st.value().accelerated == 2 && st.value().declined == 2, "stats count the outcomes");
    }
    {
        // Destroying the accelerator returned every byte to the Governor.
        safety::ResourceGovernor g(limits(64 * MiB, 16 * MiB));
        {
            auto created = vastloom::hip::HipMatvecAccelerator::create(g, options(2 * MiB), backend);
            if (!created) return 1;
            auto acc = created.take_value();
            auto m = matrix(type, rows, cols, random_blocks(type, rows, cols, rng), 0x61);
            auto y = sentinel(rows);
            (void)acc->matvec(m, x, y);
        }
        check(reserved(g, safety::ResourceKind::vram) == 0 && reserved(g, safety::ResourceKind::staging) == 0,
              "destroy returns every reservation");
    }
    {
        // Room for the scratch slots but not the matrix: declined, nothing more charged.
        const std::uint64_t tiny = 2 * MiB + 32 * 1024;
        safety::ResourceGovernor g(limits(tiny, 16 * MiB));
        auto created = vastloom::hip::HipMatvecAccelerator::create(g, options(2 * MiB), backend);
        check(created.ok(), "create within a tight VRAM budget", created.ok() ? "" : created.error().message);
        if (!created) return 1;
        auto acc = created.take_value();
        auto m = matrix(type, rows, cols, random_blocks(type, rows, cols, rng), 0x71);
        auto y = sentinel(rows);
        auto r = acc->matvec(m, x, y);
        check(r.ok() && !r.value() && untouched(y) && reserved(g, safety::ResourceKind::vram) == 2 * MiB,
              "over the Governor's VRAM budget: declined, nothing charged");
    }
    {
        // experts_only declines recurring (trunk) weights.
        safety::ResourceGovernor g(limits(64 * MiB, 16 * MiB));
        auto o = options(2 * MiB);
        o.experts_only = 1;
        auto created = vastloom::hip::HipMatvecAccelerator::create(g, o, backend);
        if (!created) return 1;
        auto acc = created.take_value();
        auto m = matrix(type, rows, cols, random_blocks(type, rows, cols, rng), 0x81, true);
        auto y = sentinel(rows);
        auto r = acc->matvec(m, x, y);
        check(r.ok() && !r.value() && untouched(y), "experts_only declines recurring weights");
    }
    if (fake_device) {
        // A failed upload is an error, not a decline, and leaves nothing resident or charged.
        safety::ResourceGovernor g(limits(64 * MiB, 16 * MiB));
        auto created = vastloom::hip::HipMatvecAccelerator::create(g, options(2 * MiB), backend);
        if (!created) return 1;
        auto acc = created.take_value();
        fake.fail_upload = true;
        auto m = matrix(type, rows, cols, random_blocks(type, rows, cols, rng), 0x91);
        auto y = sentinel(rows);
        auto r = acc->matvec(m, x, y);
        fake.fail_upload = false;
        check(!r.ok() && untouched(y) && !acc->holds(0x91) && reserved(g, safety::ResourceKind::vram) == 2 * MiB,
              "failed upload is an error, nothing resident or charged",
              r.ok() ? "not an error" : r.error().message);
    }
    std::printf("%s: %d failure(s)\n", mode, failures);
    return failures ? 1 : 0;
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "fake";
    if (mode != "fake" && mode != "hip") {
        std::printf("usage: accel_binding fake|hip\n");
        return 2;
    }
    return run(mode == "fake");
}
