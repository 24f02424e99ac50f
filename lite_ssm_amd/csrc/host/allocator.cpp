// allocator.cpp — DeviceBuffer / UnifiedBuffer for the HIP backend.
//
// Interface: include/lite_ssm/allocator.hpp (reference include/lite_ssm/allocator.hpp).
// MmapFile is not part of the backend: it is portable POSIX code and stays the
// reference's own (src/core/allocator.cpp:31-99), linked beside this library.
// The Metal bridge (src/backend/metal/metal_buffer.mm) becomes:
//   DeviceBuffer  -> HBM (lssm_malloc), so kernels run at device speed, with
//                    contents() a page-protected host mirror kept coherent at
//                    op boundaries (below); metal_buffer() is the HBM pointer.
//   UnifiedBuffer -> lssm_malloc + one upload of the whole mapping into HBM
//                    (the GPU never reads weights across PCIe); contents()
//                    stays the mmap base, as the reference's tests require.
//
// The reference's buffers are shared memory (metal_buffer.mm:120-143): its
// model layer writes embedding rows into contents() and reads the logits back
// from it between command buffers (mamba2_model.cpp:130-136,176-181).  On a
// discrete GPU the same contract is kept by a host mirror of each buffer,
// whose pages start inaccessible:
//   - a host access to an inaccessible page (SIGSEGV inside a mirror) copies
//     a window of up to 16 such pages from HBM and maps them read-only; a
//     write makes its page writable and marks it dirty;
//   - every MetalOps op, before it enqueues work on a buffer, uploads that
//     buffer's dirty pages and makes its whole mirror inaccessible again (the
//     op may change any byte of it): mirror_sync_for_device below;
//   - zero() clears the HBM copy.
// So the host reads what the GPU wrote once that work has finished (after
// commit_and_wait, or after an op outside a batch, which waits), and the GPU
// reads what the host wrote before the op was issued, as with shared memory.
// A mirror page that is inaccessible must not be handed to a system call
// (read(2), write(2) and the like report EFAULT instead of faulting): touch it
// first.  Buffers that the GPU is using must not be read or written by the
// host, exactly as with the reference's shared buffers.

#include "lite_ssm/allocator.hpp"
#include "lssm.h"
#include "mirror.hpp"

#include <signal.h>
#include <sys/mman.h>
#include <ucontext.h>
#include <unistd.h>

#include <atomic>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>

namespace lite_ssm {

namespace {

[[noreturn]] void throw_lssm(const char* what) {
    throw std::runtime_error(std::string(what) + ": " + lssm_last_error());
}

// ---- host mirrors of DeviceBuffers ----
enum : std::uint8_t { PAGE_INVALID = 0, PAGE_CLEAN = 1, PAGE_DIRTY = 2 };
constexpr int         kSlots  = 1024;   // live DeviceBuffers
constexpr std::size_t kWindow = 16;     // pages copied in per fault

// A registry entry.  Entries are never freed, only reused, so a lookup that
// races with another buffer's destruction reads a live object; every use
// re-checks `live` and the addresses under `mu`.
struct Mirror {
    std::atomic<bool>        live{false};
    std::atomic<char*>       host{nullptr};    // mmap'd, npages * page bytes
    std::atomic<char*>       dev{nullptr};     // lssm_malloc'd, same size
    std::atomic<std::size_t> npages{0};
    std::size_t              nvalid = 0;       // pages not PAGE_INVALID (under mu)
    std::uint8_t*            st     = nullptr; // per page state (under mu)
    std::mutex               mu;
};

std::atomic<Mirror*> g_slot[kSlots];
std::atomic<long>    g_valid{0};        // valid pages over every mirror
std::size_t          g_page = 4096;
lssm_ctx*            g_ctx  = nullptr;  // the mirrors' copies (never destroyed)
std::mutex           g_ctx_mu;
struct sigaction     g_prev;
std::once_flag       g_once;
bool                 g_ready = false;

bool copy(void* dst, const void* src, std::size_t n, bool to_device) {
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    return (to_device ? lssm_memcpy_h2d(g_ctx, dst, src, n) : lssm_memcpy_d2h(g_ctx, dst, src, n)) == LSSM_OK;
}

bool holds(const Mirror& m, const char* a) {
    const char* h = m.host.load(std::memory_order_acquire);
    return m.live.load(std::memory_order_acquire) && h && a >= h &&
           a < h + m.npages.load(std::memory_order_acquire) * g_page;
}

Mirror* find_host(const char* a) {
    for (auto& sl : g_slot) {
        Mirror* m = sl.load(std::memory_order_acquire);
        if (m && holds(*m, a)) return m;
    }
    return nullptr;
}

Mirror* find_dev(const void* d) {
    for (auto& sl : g_slot) {
        Mirror* m = sl.load(std::memory_order_acquire);
        if (m && m->live.load(std::memory_order_acquire) && m->dev.load(std::memory_order_acquire) == d) return m;
    }
    return nullptr;
}

// make pages [a, b) of m inaccessible (caller holds m.mu); a failure (the
// process out of memory mappings) is an error, not a stale host view
void invalidate(Mirror& m, std::size_t a, std::size_t b) {
    std::size_t n = 0;
    for (std::size_t i = a; i < b; ++i)
        if (m.st[i] != PAGE_INVALID) ++n;
    if (n == 0) return;
    if (mprotect(m.host.load() + a * g_page, (b - a) * g_page, PROT_NONE) != 0)
        throw std::runtime_error("DeviceBuffer: cannot protect the host view (mprotect failed)");
    for (std::size_t i = a; i < b; ++i) m.st[i] = PAGE_INVALID;
    m.nvalid -= n;
    g_valid.fetch_sub((long)n, std::memory_order_acq_rel);
}

// The host touched page p of m: bring it (and up to kWindow - 1 following
// invalid pages) in from HBM; a write makes page p writable and dirty.
bool fault_in(Mirror& m, const char* a, bool write) {
    std::lock_guard<std::mutex> lk(m.mu);
    if (!holds(m, a)) return false;   // destroyed meanwhile: not a mirror access any more
    const std::size_t p = (std::size_t)(a - m.host.load()) / g_page, np = m.npages.load();
    char* h = m.host.load() + p * g_page;
    if (m.st[p] == PAGE_INVALID) {
        std::size_t e = p;
        while (e < np && e - p < kWindow && m.st[e] == PAGE_INVALID) ++e;
        const std::size_t n = (e - p) * g_page;
        if (mprotect(h, n, PROT_READ | PROT_WRITE) != 0) return false;
        if (!copy(h, m.dev.load() + p * g_page, n, false)) {
            mprotect(h, n, PROT_NONE);
            return false;
        }
        for (std::size_t i = p; i < e; ++i) m.st[i] = PAGE_CLEAN;
        m.nvalid += e - p;
        g_valid.fetch_add((long)(e - p), std::memory_order_acq_rel);
        if (write) {
            m.st[p] = PAGE_DIRTY;
            if (e - p > 1) mprotect(h + g_page, n - g_page, PROT_READ);
        } else {
            mprotect(h, n, PROT_READ);
        }
        return true;
    }
    if (m.st[p] == PAGE_CLEAN && write) {
        if (mprotect(h, g_page, PROT_READ | PROT_WRITE) != 0) return false;
        m.st[p] = PAGE_DIRTY;
    }
    return true;   // (already writable: another thread brought it in)
}

// A fault on a mirror page is synchronous: the faulting thread's own load or
// store in code outside this library (the library touches mirror pages only
// after making them accessible).  So the handler may take the mirror's lock
// and call HIP as that thread could at that instruction.
void on_segv(int sig, siginfo_t* si, void* uc) {
    if (Mirror* m = find_host(static_cast<const char*>(si->si_addr))) {
        bool write = true;   // (without the fault's error code every touch counts as a write)
#if defined(__x86_64__)
        write = (static_cast<ucontext_t*>(uc)->uc_mcontext.gregs[REG_ERR] & 2) != 0;
#endif
        if (fault_in(*m, static_cast<const char*>(si->si_addr), write)) return;   // the access runs again
    }
    // not a mirror page (or its copy failed): the previous disposition
    if (g_prev.sa_flags & SA_SIGINFO) {
        if (g_prev.sa_sigaction) {
            g_prev.sa_sigaction(sig, si, uc);
            return;
        }
    } else if (g_prev.sa_handler != SIG_DFL && g_prev.sa_handler != SIG_IGN) {
        g_prev.sa_handler(sig);
        return;
    }
    signal(sig, SIG_DFL);   // the access faults again, with the default action
}

void init_mirrors() {
    std::call_once(g_once, [] {
        const long pg = sysconf(_SC_PAGESIZE);
        if (pg > 0) g_page = (std::size_t)pg;
        if (lssm_ctx_create(&g_ctx, nullptr) != LSSM_OK) return;
        // one copy each way between pageable host memory and HBM now, so that
        // the copy path's own set-up does not land in the first fault
        const std::size_t wb = kWindow * g_page;
        void* d = nullptr;
        void* h = mmap(nullptr, wb, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
        if (h == MAP_FAILED) return;
        const bool warm = lssm_malloc(&d, wb) == LSSM_OK && d && lssm_memcpy_h2d(g_ctx, d, h, wb) == LSSM_OK &&
                          lssm_memcpy_d2h(g_ctx, h, d, wb) == LSSM_OK;
        if (d) lssm_free(d);
        munmap(h, wb);
        if (!warm) return;
        struct sigaction sa;
        std::memset(&sa, 0, sizeof sa);
        sa.sa_sigaction = on_segv;
        sa.sa_flags     = SA_SIGINFO;
        sigemptyset(&sa.sa_mask);
        if (sigaction(SIGSEGV, &sa, &g_prev) != 0) return;
        g_ready = true;
    });
    if (!g_ready) throw_lssm("DeviceBuffer: host mirror set-up");
}

}  // namespace

namespace detail {

void mirror_sync_for_device(const void* handle) {
    if (!handle || g_valid.load(std::memory_order_acquire) == 0) return;
    Mirror* m = find_dev(handle);
    if (!m) return;
    std::lock_guard<std::mutex> lk(m->mu);
    if (!m->live.load() || m->dev.load() != handle || m->nvalid == 0) return;
    const std::size_t np = m->npages.load();
    char *dev = m->dev.load(), *host = m->host.load();
    for (std::size_t i = 0; i < np;) {
        if (m->st[i] != PAGE_DIRTY) {
            ++i;
            continue;
        }
        std::size_t e = i;
        while (e < np && m->st[e] == PAGE_DIRTY) ++e;
        if (!copy(dev + i * g_page, host + i * g_page, (e - i) * g_page, true))
            throw_lssm("DeviceBuffer: upload of host writes");
        i = e;
    }
    invalidate(*m, 0, np);
}

}  // namespace detail

// ---------------------------------------------------------------------------
// DeviceBuffer
// ---------------------------------------------------------------------------
DeviceBuffer::DeviceBuffer(std::size_t nbytes) {
    if (nbytes == 0) return;
    init_mirrors();
    const std::size_t np = (nbytes + g_page - 1) / g_page, bytes = np * g_page;
    void* h = mmap(nullptr, bytes, PROT_NONE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (h == MAP_FAILED) throw std::runtime_error("DeviceBuffer: mmap of the host view failed");
    void* d = nullptr;
    bool ok = lssm_malloc(&d, bytes) == LSSM_OK && d;
    if (ok) {   // zero-filled, like a new shared buffer
        std::lock_guard<std::mutex> lc(g_ctx_mu);
        ok = lssm_memset(g_ctx, d, 0, bytes) == LSSM_OK;
    }
    if (!ok) {
        const std::string why = lssm_last_error();
        if (d) lssm_free(d);
        munmap(h, bytes);
        throw std::runtime_error("DeviceBuffer: " + why);
    }
    // an entry not in use (reused), else a new one in an empty slot
    Mirror* m = nullptr;
    for (int i = 0; i < kSlots && !m; ++i) {
        Mirror* e = g_slot[i].load(std::memory_order_acquire);
        if (!e) {
            auto* fresh = new Mirror;
            fresh->live.store(true);
            Mirror* expect = nullptr;
            if (g_slot[i].compare_exchange_strong(expect, fresh, std::memory_order_acq_rel)) m = fresh;
            else delete fresh;
        } else {
            bool expect = false;
            if (e->live.compare_exchange_strong(expect, true, std::memory_order_acq_rel)) m = e;
        }
    }
    if (!m) {
        lssm_free(d);
        munmap(h, bytes);
        throw std::runtime_error("DeviceBuffer: more than 1024 live DeviceBuffers");
    }
    {
        std::lock_guard<std::mutex> lk(m->mu);
        m->st     = new std::uint8_t[np]();
        m->nvalid = 0;
        m->npages.store(np, std::memory_order_release);
        m->dev.store(static_cast<char*>(d), std::memory_order_release);
        m->host.store(static_cast<char*>(h), std::memory_order_release);
    }
    buffer_   = d;
    contents_ = h;
    length_   = nbytes;
}

DeviceBuffer::~DeviceBuffer() { reset_(); }

DeviceBuffer::DeviceBuffer(DeviceBuffer&& o) noexcept
    : buffer_(o.buffer_), contents_(o.contents_), length_(o.length_) {
    o.buffer_ = o.contents_ = nullptr;
    o.length_ = 0;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
        reset_();
        buffer_   = o.buffer_;
        contents_ = o.contents_;
        length_   = o.length_;
        o.buffer_ = o.contents_ = nullptr;
        o.length_ = 0;
    }
    return *this;
}

void DeviceBuffer::zero() {
    Mirror* m = buffer_ ? find_dev(buffer_) : nullptr;
    if (!m) return;
    std::lock_guard<std::mutex> lk(m->mu);
    int rc;
    {
        std::lock_guard<std::mutex> lc(g_ctx_mu);
        rc = lssm_memset(g_ctx, m->dev.load(), 0, m->npages.load() * g_page);
    }
    if (rc != LSSM_OK) throw_lssm("DeviceBuffer::zero");
    invalidate(*m, 0, m->npages.load());
}

void DeviceBuffer::reset_() noexcept {
    if (buffer_) {
        if (Mirror* m = find_dev(buffer_)) {
            std::lock_guard<std::mutex> lk(m->mu);
            const std::size_t np = m->npages.load();
            m->live.store(false, std::memory_order_release);
            g_valid.fetch_sub((long)m->nvalid, std::memory_order_acq_rel);
            munmap(m->host.load(), np * g_page);
            lssm_free(m->dev.load());
            delete[] m->st;
            m->st     = nullptr;
            m->nvalid = 0;
            m->host.store(nullptr);
            m->dev.store(nullptr);
            m->npages.store(0);
        }
    }
    buffer_ = contents_ = nullptr;
    length_ = 0;
}

// ---------------------------------------------------------------------------
// UnifiedBuffer
// ---------------------------------------------------------------------------
UnifiedBuffer::UnifiedBuffer(const MmapFile& mapping) {
    if (!mapping.valid()) throw std::runtime_error("UnifiedBuffer: source MmapFile is empty");
    void* dev = nullptr;
    if (lssm_malloc(&dev, mapping.mapped_size()) != LSSM_OK || !dev) throw_lssm("UnifiedBuffer");
    lssm_ctx* ctx = nullptr;
    if (lssm_ctx_create(&ctx, nullptr) != LSSM_OK) {
        lssm_free(dev);
        throw_lssm("UnifiedBuffer");
    }
    const int rc = lssm_memcpy_h2d(ctx, dev, mapping.data(), mapping.file_size());
    lssm_ctx_destroy(ctx);
    if (rc != LSSM_OK) {
        lssm_free(dev);
        throw_lssm("UnifiedBuffer: upload");
    }
    buffer_   = dev;
    contents_ = mapping.data();
    length_   = mapping.mapped_size();
}

UnifiedBuffer::~UnifiedBuffer() { reset_(); }

UnifiedBuffer::UnifiedBuffer(UnifiedBuffer&& o) noexcept
    : buffer_(o.buffer_), contents_(o.contents_), length_(o.length_) {
    o.buffer_   = nullptr;
    o.contents_ = nullptr;
    o.length_   = 0;
}

UnifiedBuffer& UnifiedBuffer::operator=(UnifiedBuffer&& o) noexcept {
    if (this != &o) {
        reset_();
        buffer_     = o.buffer_;
        contents_   = o.contents_;
        length_     = o.length_;
        o.buffer_   = nullptr;
        o.contents_ = nullptr;
        o.length_   = 0;
    }
    return *this;
}

void UnifiedBuffer::reset_() noexcept {
    if (buffer_) lssm_free(buffer_);
    buffer_   = nullptr;
    contents_ = nullptr;
    length_   = 0;
}

}  // namespace lite_ssm
