#pragma once

#include <cstddef>
#include <memory>

#include "core/status.hpp"
#include "scicompute_attention/export.hpp"

namespace sci {
class Device;
}  // namespace sci

namespace sca {

// Interface of the reference's Workspace (include/scicompute_attention/workspace.hpp:17-50).
//
// One device allocation made at Create(), handed out as caller-placed slices: a slice must be
// `align`-aligned, lie inside the buffer and either not overlap any earlier slice or repeat one
// exactly. Reset() forgets the slices and keeps the memory. Copies share the buffer.
class SCI_ATTENTION_API Workspace {
public:
    Workspace();
    Workspace(const Workspace&) = default;
    Workspace& operator=(const Workspace&) = default;
    ~Workspace();

    static sci::Result<Workspace> Create(size_t bytes, sci::Device& device);

    void* Data() noexcept;
    const void* Data() const noexcept;
    size_t Bytes() const noexcept;
    bool Valid() const noexcept;

    sci::Result<void*> Slice(size_t offset, size_t bytes, size_t align = 256);
    sci::Status Reset();

    size_t PeakBytes() const noexcept;
    size_t AllocatedSlices() const noexcept;

private:
    struct Impl;
    std::shared_ptr<Impl> impl_;
};

}  // namespace sca
