// Owning device and pinned host buffers (the roles of include/zcgvs/core/device_buffer.hpp:40-56
// and pinned_buffer.hpp), allocated through the C ABI. Move-only; contents are uninitialized.
#pragma once

#include <cstddef>
#include <utility>

#include "zcgvs/core/error.hpp"

namespace zcgvs {

template <typename T>
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(std::size_t count) { allocate(count); }
    ~DeviceBuffer() { release(); }

    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& other) noexcept { swap(other); }
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept {
        if (this != &other) {
            release();
            swap(other);
        }
        return *this;
    }

    // Replaces the allocation with one of `count` elements (previous contents are dropped).
    void allocate(std::size_t count) {
        release();
        if (count == 0) {
            return;
        }
        void* pointer = nullptr;
        check(zcgvs_malloc(&pointer, count * sizeof(T)));
        data_ = static_cast<T*>(pointer);
        size_ = count;
    }

    void release() noexcept {
        if (data_ != nullptr) {
            zcgvs_free(data_);
        }
        data_ = nullptr;
        size_ = 0;
    }

    void copyFromHost(const T* host, std::size_t count, zcgvs_stream_t stream, std::size_t offset = 0) {
        check(zcgvs_memcpy_h2d(data_ + offset, host, count * sizeof(T), stream));
    }
    void copyToHost(T* host, std::size_t count, zcgvs_stream_t stream, std::size_t offset = 0) const {
        check(zcgvs_memcpy_d2h(host, data_ + offset, count * sizeof(T), stream));
    }

    T* data() { return data_; }
    const T* data() const { return data_; }
    std::size_t size() const { return size_; }
    std::size_t bytes() const { return size_ * sizeof(T); }

private:
    void swap(DeviceBuffer& other) noexcept {
        std::swap(data_, other.data_);
        std::swap(size_, other.size_);
    }

    T* data_ = nullptr;
    std::size_t size_ = 0;
};

template <typename T>
class PinnedBuffer {
public:
    PinnedBuffer() = default;
    explicit PinnedBuffer(std::size_t count) { allocate(count); }
    ~PinnedBuffer() { release(); }

    PinnedBuffer(const PinnedBuffer&) = delete;
    PinnedBuffer& operator=(const PinnedBuffer&) = delete;
    PinnedBuffer(PinnedBuffer&& other) noexcept { swap(other); }
    PinnedBuffer& operator=(PinnedBuffer&& other) noexcept {
        if (this != &other) {
            release();
            swap(other);
        }
        return *this;
    }

    void allocate(std::size_t count) {
        release();
        if (count == 0) {
            return;
        }
        void* pointer = nullptr;
        check(zcgvs_host_alloc(&pointer, count * sizeof(T)));
        data_ = static_cast<T*>(pointer);
        size_ = count;
    }

    void release() noexcept {
        if (data_ != nullptr) {
            zcgvs_host_free(data_);
        }
        data_ = nullptr;
        size_ = 0;
    }

    T* data() { return data_; }
    const T* data() const { return data_; }
    std::size_t size() const { return size_; }

private:
    void swap(PinnedBuffer& other) noexcept {
        std::swap(data_, other.data_);
        std::swap(size_, other.size_);
    }

    T* data_ = nullptr;
    std::size_t size_ = 0;
};

}  // namespace zcgvs
