// tests/cpp/test_metal_ops.cpp — the reference's tests/test_metal_ops.cpp:17-78
// run against the HIP backend, plus a numeric pass through the same C++
// interface (lite_ssm::MetalOps, DeviceBuffer, UnifiedBuffer) checked against
// the CPU oracle (oracle/liblssm_oracle.so, linked only into this test).
//
// Exit 77 (skip) when no GPU / HIP code object is available, as the reference.

#include "lite_ssm/allocator.hpp"
#include "lite_ssm/ops.hpp"

extern "C" {
#include "../../oracle/lssm_oracle.h"
}

#include <array>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <random>
#include <stdexcept>
#include <string>
#include <string_view>
#include <thread>
#include <unistd.h>
#include <vector>

namespace {

constexpr int SKIP = 77;
int g_fail = 0;

#define EXPECT(cond, ...)                                                   \
    do {                                                                    \
        if (!(cond)) {                                                      \
            std::fprintf(stderr, "FAIL %s:%d: %s — ", __FILE__, __LINE__, #cond); \
            std::fprintf(stderr, __VA_ARGS__);                              \
            std::fprintf(stderr, "\n");                                     \
            ++g_fail;                                                       \
        }                                                                   \
    } while (0)

std::mt19937 rng(1234);

std::vector<uint16_t> rand_f16(std::size_t n, float lo, float hi) {
    std::uniform_real_distribution<float> u(lo, hi);
    std::vector<uint16_t> v(n);
    for (auto& e : v) e = orc_f2h(u(rng));
    return v;
}

// max |a-b| / max(max|b|, tiny) over fp16 vectors
double max_rel16(const uint16_t* a, const uint16_t* b, std::size_t n) {
    double num = 0, den = 1e-6;
    for (std::size_t i = 0; i < n; ++i) {
        const double x = orc_h2f(a[i]), y = orc_h2f(b[i]);
        num = std::fmax(num, std::fabs(x - y));
        den = std::fmax(den, std::fabs(y));
    }
    return num / den;
}

double max_rel32(const float* a, const float* b, std::size_t n) {
    double num = 0, den = 1e-6;
    for (std::size_t i = 0; i < n; ++i) {
        num = std::fmax(num, std::fabs((double)a[i] - b[i]));
        den = std::fmax(den, std::fabs((double)b[i]));
    }
    return num / den;
}

template <class T>
T* host(lite_ssm::DeviceBuffer& b) { return static_cast<T*>(b.contents()); }

bool throws_with(const std::function<void()>& f, const char* text) {
    try {
        f();
    } catch (const std::runtime_error& e) {
        return std::strstr(e.what(), text) != nullptr;
    }
    return false;
}

}  // namespace

int main() {
    lite_ssm::MetalOps ops;
    if (!ops.metallib_loaded()) {
        std::fprintf(stderr, "[test_metal_ops] SKIP: no GPU or HIP code object not loadable\n");
        return SKIP;
    }
    std::printf("[test_metal_ops] library: %s\n", ops.metallib_path().c_str());

    // --- 1. every reference kernel name resolves (test_metal_ops.cpp:30-77) ---
    constexpr std::array<std::string_view, 17> kernels = {
        "lite_ssm_common_noop", "rmsnorm_f16", "silu_f16", "silu_gated_f16",
        "linear_f16_gemv", "linear_silu_f16_gemv", "rmsnorm_linear_f16_gemv",
        "linear_f16_gemm", "linear_silu_f16_gemm", "causal_conv1d_f16",
        "causal_conv1d_update_f16", "ssd_chunked_f16", "ssd_step_f16",
        "linear_int4_gemv", "linear_int4_gemm", "seed_conv_state_f16",
        "inproj_fused_f16",
    };
    for (auto name : kernels)
        EXPECT(ops.has_pipeline(name), "%.*s missing", (int)name.size(), name.data());
    EXPECT(!ops.has_pipeline("no_such_kernel"), "unknown name resolved");

    // --- 2. rmsnorm_f16 through DeviceBuffer handles with byte offsets --------
    {
        const uint32_t rows = 3, dim = 256;
        const float eps = 1e-5f;
        auto x = rand_f16(rows * dim, -2.f, 2.f), w = rand_f16(dim, 0.5f, 1.5f);
        lite_ssm::DeviceBuffer buf(4096 + (rows * dim * 2 + dim) * 2);
        const std::size_t xo = 256, wo = xo + rows * dim * 2, yo = wo + dim * 2;
        std::memcpy(host<uint8_t>(buf) + xo, x.data(), x.size() * 2);
        std::memcpy(host<uint8_t>(buf) + wo, w.data(), w.size() * 2);
        ops.rmsnorm_f16(buf.metal_buffer(), xo, buf.metal_buffer(), wo, buf.metal_buffer(), yo,
                        {rows, dim, eps});
        std::vector<uint16_t> ref(rows * dim);
        orc_rmsnorm(x.data(), w.data(), ref.data(), rows, dim, eps, LSSM_F16);
        const double e = max_rel16(reinterpret_cast<uint16_t*>(host<uint8_t>(buf) + yo),
                                   ref.data(), ref.size());
        EXPECT(e < 2e-2, "rmsnorm_f16 max-rel %.3g", e);
        EXPECT(throws_with([&] {
                   ops.rmsnorm_f16(buf.metal_buffer(), xo, buf.metal_buffer(), wo,
                                   buf.metal_buffer(), yo, {rows, 6, eps});
               }, "rmsnorm_f16: dim must be a multiple of 4"),
               "rmsnorm_f16 dim check");
    }

    // --- 3. linear_int4_gemv from a mmap'd weight file via UnifiedBuffer ------
    {
        const uint32_t N = 96, K = 256;
        std::vector<float> wf(N * K);
        std::normal_distribution<float> g(0.f, 0.05f);
        for (auto& v : wf) v = g(rng);
        const std::size_t pbytes = (std::size_t)N * K / 2, sbytes = (std::size_t)N * K / 32 * 2;
        std::vector<uint8_t> file(64 + pbytes + sbytes);
        orc_quantize(wf.data(), N, K, LSSM_W_Q4_B32, file.data() + 64,
                     reinterpret_cast<uint16_t*>(file.data() + 64 + pbytes));
        char path[] = "/tmp/lssm_test_weightsXXXXXX";
        const int fd = ::mkstemp(path);
        EXPECT(fd >= 0, "mkstemp");
        EXPECT(::write(fd, file.data(), file.size()) == (ssize_t)file.size(), "write");
        ::close(fd);
        {
            lite_ssm::MmapFile map(path);
            lite_ssm::UnifiedBuffer wbuf(map);
            EXPECT(wbuf.contents() == map.data(), "UnifiedBuffer contents == mmap base");
            EXPECT(wbuf.length() == map.mapped_size(), "UnifiedBuffer length == mapped_size");
            EXPECT(wbuf.metal_buffer() != nullptr, "UnifiedBuffer device handle");

            auto x = rand_f16(K, -1.f, 1.f);
            lite_ssm::DeviceBuffer io((K + N) * 2);
            std::memcpy(io.contents(), x.data(), K * 2);
            ops.linear_int4_gemv(io.metal_buffer(), 0, wbuf.metal_buffer(), 64,
                                 wbuf.metal_buffer(), 64 + pbytes, io.metal_buffer(), K * 2,
                                 {1, N, K});
            std::vector<uint16_t> ref(N);
            orc_linear(x.data(), 0, file.data() + 64, file.data() + 64 + pbytes, ref.data(), 0,
                       nullptr, 1, N, K, LSSM_W_Q4_B32, LSSM_F16, LSSM_EPI_NONE, 0);
            const double e = max_rel16(host<uint16_t>(io) + K, ref.data(), N);
            EXPECT(e < 2e-2, "linear_int4_gemv max-rel %.3g", e);
            EXPECT(throws_with([&] {
                       ops.linear_int4_gemv(io.metal_buffer(), 0, wbuf.metal_buffer(), 64,
                                            wbuf.metal_buffer(), 64 + pbytes, io.metal_buffer(),
                                            K * 2, {1, N, 40});
                   }, "K must be a multiple of 32"),
                   "linear_int4_gemv K check");
        }
        ::unlink(path);
    }

    // --- 4. a batch: ops are queued, results visible after commit_and_wait ----
    {
        const uint32_t n = 1000;
        auto a = rand_f16(n, -4.f, 4.f), b = rand_f16(n, -1.f, 1.f);
        lite_ssm::DeviceBuffer buf(3 * n * 2);
        std::memcpy(host<uint16_t>(buf), a.data(), n * 2);
        std::memcpy(host<uint16_t>(buf) + n, b.data(), n * 2);
        ops.begin_batch();
        EXPECT(ops.batch_active(), "batch_active after begin_batch");
        EXPECT(throws_with([&] { ops.begin_batch(); }, "already active"), "nested begin_batch");
        ops.silu_f16(buf.metal_buffer(), 0, buf.metal_buffer(), 2 * n * 2, n);
        ops.add_inplace_f16(buf.metal_buffer(), 2 * n * 2, buf.metal_buffer(), n * 2, n);
        ops.commit_and_wait();
        EXPECT(!ops.batch_active(), "batch inactive after commit");
        std::vector<uint16_t> ref(n);
        orc_silu(a.data(), ref.data(), n, LSSM_F16);
        orc_add_inplace(ref.data(), b.data(), n, LSSM_F16);
        const double e = max_rel16(host<uint16_t>(buf) + 2 * n, ref.data(), n);
        EXPECT(e < 2e-2, "silu+add batch max-rel %.3g", e);
        EXPECT(throws_with([&] { ops.commit_and_wait(); }, "without an active batch"),
               "commit without batch");
    }

    // --- 5. ssd_step_f16: state in a DeviceBuffer, updated in place ----------
    {
        const uint32_t H = 4, P = 64, N = 128, G = 1;
        auto x = rand_f16(H * P, -1.f, 1.f), B = rand_f16(G * N, -1.f, 1.f),
             C = rand_f16(G * N, -1.f, 1.f), dt = rand_f16(H, -3.f, 0.f),
             db = rand_f16(H, -1.f, 0.f), Al = rand_f16(H, 0.f, 2.f), D = rand_f16(H, 0.5f, 1.5f);
        std::vector<float> s0(H * P * N);
        std::uniform_real_distribution<float> u(-0.5f, 0.5f);
        for (auto& v : s0) v = u(rng);
        const std::size_t nh = x.size() + B.size() + C.size() + dt.size() + db.size() + Al.size() +
                               D.size() + H * P;
        lite_ssm::DeviceBuffer st(s0.size() * 4), hb(nh * 2);
        std::memcpy(st.contents(), s0.data(), s0.size() * 4);
        std::size_t off[8], o = 0;
        const std::vector<uint16_t>* parts[7] = {&x, &B, &C, &dt, &db, &Al, &D};
        for (int i = 0; i < 7; ++i) {
            off[i] = o * 2;
            std::memcpy(host<uint16_t>(hb) + o, parts[i]->data(), parts[i]->size() * 2);
            o += parts[i]->size();
        }
        off[7] = o * 2;
        const lite_ssm::SSDStepDims d{H, P, N, G, 0.0f, INFINITY, 1};
        void* h = hb.metal_buffer();
        ops.ssd_step_f16(h, off[0], h, off[1], h, off[2], h, off[3], h, off[4], h, off[5], h,
                         off[6], st.metal_buffer(), 0, h, off[7], d);
        std::vector<float> sref = s0;
        std::vector<uint16_t> yref(H * P);
        orc_ssd_step(x.data(), B.data(), C.data(), dt.data(), db.data(), Al.data(), D.data(),
                     sref.data(), yref.data(), 1,
                     lssm_ssd_step_dims{H, P, N, G, 0.0f, INFINITY, 1}, LSSM_F16);
        const double ey = max_rel16(host<uint16_t>(hb) + o, yref.data(), yref.size());
        const double es = max_rel32(host<float>(st), sref.data(), sref.size());
        EXPECT(ey < 2e-2, "ssd_step y max-rel %.3g", ey);
        EXPECT(es < 1e-3, "ssd_step state max-rel %.3g", es);
    }

    // --- 6. DeviceBuffer's host view (HBM storage, page-protected mirror) ---
    // host writes reach the op, the op's writes reach later host reads, over
    // pages brought in as windows, rewritten after a read, cleared by zero(),
    // across two buffers and after a move
    {
        const uint32_t n = 20000;                     // 40 KB per fp16 vector: 10 pages
        const std::size_t pg = (std::size_t)sysconf(_SC_PAGESIZE);
        lite_ssm::DeviceBuffer buf(3 * n * 2 + 6);    // not a whole number of pages
        bool zero0 = true;                            // a new buffer reads as zeros
        for (uint32_t i = 0; i < 3 * n; ++i) zero0 = zero0 && host<uint16_t>(buf)[i] == 0;
        EXPECT(zero0, "new DeviceBuffer reads zero");
        for (int pass = 0; pass < 3; ++pass) {
            auto a = rand_f16(n, -4.f, 4.f), b = rand_f16(n, -1.f, 1.f);
            // pass 1 rewrites pages the host has just read (clean -> dirty);
            // pass 2 writes one element per page only, the rest stays as read
            if (pass < 2) {
                std::memcpy(host<uint16_t>(buf), a.data(), n * 2);
                std::memcpy(host<uint16_t>(buf) + n, b.data(), n * 2);
            } else {
                for (uint32_t i = 0; i < n; ++i) {
                    a[i] = host<uint16_t>(buf)[i];
                    b[i] = host<uint16_t>(buf)[n + i];
                }
                for (uint32_t i = 0; i < n; i += (uint32_t)(pg / 2)) {
                    a[i] = orc_f2h(0.5f + i % 7);
                    host<uint16_t>(buf)[i] = a[i];
                }
            }
            ops.silu_f16(buf.metal_buffer(), 0, buf.metal_buffer(), 2 * n * 2, n);
            ops.add_inplace_f16(buf.metal_buffer(), 2 * n * 2, buf.metal_buffer(), n * 2, n);
            std::vector<uint16_t> ref(n);
            orc_silu(a.data(), ref.data(), n, LSSM_F16);
            orc_add_inplace(ref.data(), b.data(), n, LSSM_F16);
            const double e = max_rel16(host<uint16_t>(buf) + 2 * n, ref.data(), n);
            EXPECT(e < 2e-2, "host view pass %d: silu+add max-rel %.3g", pass, e);
        }
        // the last bytes, past the last whole page, round-trip too
        host<uint8_t>(buf)[3 * n * 2 + 5] = 0xA5;
        ops.silu_f16(buf.metal_buffer(), 0, buf.metal_buffer(), 2 * n * 2, 1);
        EXPECT(host<uint8_t>(buf)[3 * n * 2 + 5] == 0xA5, "tail byte kept across an op");
        buf.zero();
        bool zeroed = true;
        for (uint32_t i = 0; i < 3 * n; ++i) zeroed = zeroed && host<uint16_t>(buf)[i] == 0;
        EXPECT(zeroed, "zero() clears what the host sees");
        // two buffers: input in one, output in the other; then the buffer moved
        lite_ssm::DeviceBuffer in(n * 2), out(n * 2);
        auto a = rand_f16(n, -4.f, 4.f);
        std::memcpy(host<uint16_t>(in), a.data(), n * 2);
        std::memset(host<uint16_t>(out), 0x3C, n * 2);     // overwritten by the op
        ops.silu_f16(in.metal_buffer(), 0, out.metal_buffer(), 0, n);
        lite_ssm::DeviceBuffer moved(std::move(out));
        std::vector<uint16_t> ref(n);
        orc_silu(a.data(), ref.data(), n, LSSM_F16);
        const double e = max_rel16(host<uint16_t>(moved), ref.data(), n);
        EXPECT(e < 2e-2, "two buffers: silu max-rel %.3g", e);
        EXPECT(std::memcmp(host<uint16_t>(in), a.data(), n * 2) == 0, "input kept");
    }

    // --- 8. repeated batches, as the model layer's decode steps issue them:
    // the same ops on the same buffers with new host data each time, and
    // batches of other sizes in between, every result checked
    {
        const uint32_t n = 6000;
        lite_ssm::DeviceBuffer buf(3 * n * 2);
        const uint32_t sizes[] = {n, n, n, n, n, n / 2, n / 2, n, n, n, n};
        for (std::size_t it = 0; it < sizeof(sizes) / sizeof(sizes[0]); ++it) {
            const uint32_t m = sizes[it];
            auto a = rand_f16(m, -4.f, 4.f), b = rand_f16(m, -1.f, 1.f);
            std::memcpy(host<uint16_t>(buf), a.data(), m * 2);
            std::memcpy(host<uint16_t>(buf) + n, b.data(), m * 2);
            ops.begin_batch();
            ops.silu_f16(buf.metal_buffer(), 0, buf.metal_buffer(), 2 * n * 2, m);
            ops.add_inplace_f16(buf.metal_buffer(), 2 * n * 2, buf.metal_buffer(), n * 2, m);
            ops.commit_and_wait();
            std::vector<uint16_t> ref(m);
            orc_silu(a.data(), ref.data(), m, LSSM_F16);
            orc_add_inplace(ref.data(), b.data(), m, LSSM_F16);
            const double e = max_rel16(host<uint16_t>(buf) + 2 * n, ref.data(), m);
            EXPECT(e < 2e-2, "repeated batch %zu (n %u): silu+add max-rel %.3g", it, m, e);
        }
    }

    // --- 7. host views from several threads at once: each thread its own
    // MetalOps, buffers created, written, run, read and destroyed in a loop
    // (registry entries reused while other threads look them up)
    {
        constexpr int kThreads = 4, kIters = 12;
        std::atomic<int> bad{0};
        std::vector<std::thread> th;
        for (int t = 0; t < kThreads; ++t) {
            th.emplace_back([t, &bad] {
                try {
                    lite_ssm::MetalOps tops;
                    std::mt19937 r(100 + t);
                    std::uniform_real_distribution<float> u(-4.f, 4.f);
                    for (int it = 0; it < kIters; ++it) {
                        const uint32_t n = 3000 + 1000 * (uint32_t)((t + it) % 5);
                        std::vector<uint16_t> a(n), ref(n);
                        for (auto& e : a) e = orc_f2h(u(r));
                        lite_ssm::DeviceBuffer b(2 * n * 2);
                        std::memcpy(b.contents(), a.data(), n * 2);
                        tops.silu_f16(b.metal_buffer(), 0, b.metal_buffer(), n * 2, n);
                        orc_silu(a.data(), ref.data(), n, LSSM_F16);
                        if (max_rel16(static_cast<const uint16_t*>(b.contents()) + n, ref.data(), n) >= 2e-2)
                            bad.fetch_add(1);
                    }
                } catch (const std::exception& e) {
                    std::fprintf(stderr, "thread %d: %s\n", t, e.what());
                    bad.fetch_add(1);
                }
            });
        }
        for (auto& x : th) x.join();
        EXPECT(bad.load() == 0, "%d of %d threaded iterations wrong", bad.load(), kThreads * kIters);
    }

    if (g_fail) {
        std::fprintf(stderr, "[test_metal_ops] FAIL: %d check(s)\n", g_fail);
        return 1;
    }
    std::printf("[test_metal_ops] OK: all %zu kernels present, numeric checks pass\n",
                kernels.size());
    return 0;
}
