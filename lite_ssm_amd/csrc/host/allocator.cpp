// allocator.cpp — DeviceBuffer / UnifiedBuffer for the HIP backend.
//
// Interface: include/lite_ssm/allocator.hpp (reference include/lite_ssm/allocator.hpp).
// MmapFile is not part of the backend: it is portable POSIX code and stays the
// reference's own (src/core/allocator.cpp:31-99), linked beside this library.
// The Metal bridge (src/backend/metal/metal_buffer.mm) becomes:
//   DeviceBuffer  -> lssm_malloc_host: pinned, coherent host memory mapped
//                    into the GPU, so the model layer's contents() reads and
//                    writes (embedding rows in, logits out) keep working with no
//                    copies; metal_buffer() == contents() == that pointer.
//                    Kernels reach it over PCIe: this keeps the reference's
//                    model layer correct, and the HBM-resident path is the
//                    engine (lssm_engine_*), which allocates with lssm_malloc.
//   UnifiedBuffer -> lssm_malloc + one upload of the whole mapping into HBM
//                    (the GPU never reads weights across PCIe); contents()
//                    stays the mmap base, as the reference's tests require.

#include "lite_ssm/allocator.hpp"
#include "lssm.h"

#include <cstring>
#include <stdexcept>
#include <string>

namespace lite_ssm {

namespace {

[[noreturn]] void throw_lssm(const char* what) {
    throw std::runtime_error(std::string(what) + ": " + lssm_last_error());
}

}  // namespace

// ---------------------------------------------------------------------------
// DeviceBuffer
// ---------------------------------------------------------------------------
DeviceBuffer::DeviceBuffer(std::size_t nbytes) {
    if (nbytes == 0) return;
    void* p = nullptr;
    if (lssm_malloc_host(&p, nbytes) != LSSM_OK || !p) throw_lssm("DeviceBuffer");
    buffer_   = p;
    contents_ = p;
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
    if (contents_ && length_) std::memset(contents_, 0, length_);
}

void DeviceBuffer::reset_() noexcept {
    if (buffer_) lssm_free_host(buffer_);
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
