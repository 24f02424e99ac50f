#pragma once
// lite_ssm/allocator.hpp — memory plumbing of the HIP backend.
//
// Same public interface as the reference's include/lite_ssm/allocator.hpp
// (MmapFile :21-44, DeviceBuffer :49-73, UnifiedBuffer :75-103) so that the
// model layer compiles unchanged against it.  On a discrete MI355X:
//
//   MmapFile      POSIX mmap(PROT_READ, MAP_PRIVATE) of a whole file.
//   DeviceBuffer  HBM (metal_buffer(), the kernels' pointer) with a host
//                 mirror as contents(): the CPU view the model layer memcpy's
//                 into (embed) and reads logits from.  Mirror pages are
//                 brought in from HBM when the host touches them and written
//                 back before the next op that names the buffer, so the host
//                 sees the GPU's writes once that work has finished, as with
//                 the reference's shared buffers.  An inaccessible mirror page
//                 must be touched before it is passed to a system call.
//   UnifiedBuffer the weights: an HBM copy of the mapping uploaded once;
//                 contents() stays the mmap base (reference contract,
//                 tests/test_mmap_loader.cpp:99-103), metal_buffer() is the
//                 device pointer, so (metal_buffer() + tensor offset) addresses
//                 the tensor in HBM.

#include <cstddef>
#include <string>

namespace lite_ssm {

class MmapFile {
public:
    MmapFile() = default;
    explicit MmapFile(const std::string& path);
    ~MmapFile();

    MmapFile(const MmapFile&)            = delete;
    MmapFile& operator=(const MmapFile&) = delete;
    MmapFile(MmapFile&& other) noexcept;
    MmapFile& operator=(MmapFile&& other) noexcept;

    const void*  data()        const { return ptr_; }
    std::size_t  file_size()   const { return file_size_; }
    std::size_t  mapped_size() const { return mapped_size_; }
    bool         valid()       const { return ptr_ != nullptr; }

private:
    void        reset_() noexcept;

    void*       ptr_         = nullptr;
    std::size_t file_size_   = 0;
    std::size_t mapped_size_ = 0;
};

class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(std::size_t nbytes);
    ~DeviceBuffer();

    DeviceBuffer(const DeviceBuffer&)            = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&&) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&&) noexcept;

    void*       metal_buffer() const { return buffer_; }     // device pointer (kernel handle)
    void*       contents()     const { return contents_; }   // CPU pointer
    std::size_t length()       const { return length_; }
    bool        valid()        const { return buffer_ != nullptr; }

    void zero();   // memset(contents, 0, length) — for state reset

private:
    void reset_() noexcept;

    void*       buffer_   = nullptr;
    void*       contents_ = nullptr;
    std::size_t length_   = 0;
};

class UnifiedBuffer {
public:
    UnifiedBuffer() = default;
    explicit UnifiedBuffer(const MmapFile& mapping);
    ~UnifiedBuffer();

    UnifiedBuffer(const UnifiedBuffer&)            = delete;
    UnifiedBuffer& operator=(const UnifiedBuffer&) = delete;
    UnifiedBuffer(UnifiedBuffer&& other) noexcept;
    UnifiedBuffer& operator=(UnifiedBuffer&& other) noexcept;

    void*        metal_buffer() const { return buffer_; }   // HBM copy of the mapping
    const void*  contents()     const { return contents_; } // == MmapFile::data()
    std::size_t  length()       const { return length_; }
    bool         valid()        const { return buffer_ != nullptr; }

private:
    void        reset_() noexcept;

    void*       buffer_   = nullptr;
    const void* contents_ = nullptr;
    std::size_t length_   = 0;
};

}  // namespace lite_ssm
