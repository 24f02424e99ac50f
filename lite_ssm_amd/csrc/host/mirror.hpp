#pragma once
// mirror.hpp — the coherence hook between MetalOps and DeviceBuffer's host
// mirror (allocator.cpp).

namespace lite_ssm::detail {

// Before an op enqueues work on the buffer whose device handle is `handle`:
// upload the host's writes to its mirror and make the mirror inaccessible, so
// that host reads after the op fetch what the GPU wrote.  No-op for handles
// that are not DeviceBuffers (UnifiedBuffer weights) and when no mirror page
// is accessible.  Throws std::runtime_error when an upload fails.
void mirror_sync_for_device(const void* handle);

}  // namespace lite_ssm::detail
