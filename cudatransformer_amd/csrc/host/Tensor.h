// Tensor<DType>: a shape plus a shared device buffer, the allocation / transfer part of the
// reference's Tensor (Tensor.cu:11-285, headers.cu:195-237).
//
// Same ownership model as the reference: copies are shallow (shared_ptr to the device
// buffer, Tensor.cu:73-113), clone() is deep, constructors zero-fill (Tensor.cu:27-55).
// Different mechanics: buffers come from a caching allocator (BlockCache) and fills /
// copies are enqueued on the one runtime stream, instead of cudaMalloc + fill kernel +
// cudaDeviceSynchronize per allocation (headers.cu:195-215).  The
// host waits only when data comes back to the CPU (numpy(), item()) or after an upload from
// pageable memory (fromPointer()).
//
// DType is float, double, bf16 or f16 (both stored as their 16-bit patterns), or int32_t for
// token ids.  The reference's tensor algebra (Tensor.cu:290-958) is not part of this path.
#pragma once

#include <atomic>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <numeric>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "Runtime.h"

namespace ct {

// bfloat16 storage type (upper half of an IEEE binary32).
struct bf16 {
    uint16_t bits = 0;
    static bf16 fromFloat(float f) {
        uint32_t u;
        std::memcpy(&u, &f, 4);
        bf16 b;
        if ((u & 0x7fffffffu) > 0x7f800000u) {
            b.bits = uint16_t((u >> 16) | 0x40);  // quiet NaN
        } else {
            u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
            b.bits = uint16_t(u >> 16);
        }
        return b;
    }
    float toFloat() const {
        uint32_t u = uint32_t(bits) << 16;
        float f;
        std::memcpy(&f, &u, 4);
        return f;
    }
};

// IEEE binary16 storage type, converted on the host with round to nearest even (subnormals,
// infinities and NaN included).
struct f16 {
    uint16_t bits = 0;
    static f16 fromFloat(float f) {
        uint32_t x;
        std::memcpy(&x, &f, 4);
        const uint32_t sign = (x >> 16) & 0x8000u;
        uint32_t mant = x & 0x7fffffu;
        const int exp = int((x >> 23) & 0xffu);
        f16 h;
        if (exp == 255) {  // inf / NaN (NaN stays quiet)
            h.bits = uint16_t(sign | 0x7c00u | (mant ? 0x200u | (mant >> 13) : 0u));
            return h;
        }
        const int e = exp - 127 + 15;
        if (e >= 31) {
            h.bits = uint16_t(sign | 0x7c00u);
        } else if (e <= 0) {  // subnormal half, or zero
            if (e < -10) {
                h.bits = uint16_t(sign);
            } else {
                mant |= 0x800000u;
                const int shift = 14 - e;
                uint32_t v = mant >> shift;
                const uint32_t rem = mant & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
                if (rem > halfway || (rem == halfway && (v & 1u))) ++v;
                h.bits = uint16_t(sign | v);
            }
        } else {
            uint32_t v = (uint32_t(e) << 10) | (mant >> 13);
            const uint32_t rem = mant & 0x1fffu;
            if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) ++v;  // a carry may reach inf: correct
            h.bits = uint16_t(sign | v);
        }
        return h;
    }
    float toFloat() const {
        const uint32_t sign = uint32_t(bits & 0x8000u) << 16;
        uint32_t exp = (bits >> 10) & 0x1fu, mant = bits & 0x3ffu, u;
        if (exp == 0) {
            if (mant == 0) {
                u = sign;
            } else {  // subnormal: normalise
                exp = 127 - 15 + 1;
                while (!(mant & 0x400u)) {
                    mant <<= 1;
                    --exp;
                }
                u = sign | (exp << 23) | ((mant & 0x3ffu) << 13);
            }
        } else if (exp == 31) {
            u = sign | 0x7f800000u | (mant << 13);
        } else {
            u = sign | ((exp - 15 + 127) << 23) | (mant << 13);
        }
        float f;
        std::memcpy(&f, &u, 4);
        return f;
    }
};

template <typename DType> struct DTypeCode;
template <> struct DTypeCode<float> { static constexpr int value = CTATTN_F32; };
template <> struct DTypeCode<bf16> { static constexpr int value = CTATTN_BF16; };
template <> struct DTypeCode<f16> { static constexpr int value = CTATTN_F16; };
template <> struct DTypeCode<double> { static constexpr int value = CTATTN_F64; };
template <> struct DTypeCode<int32_t> { static constexpr int value = CTATTN_I32; };
template <> struct DTypeCode<int64_t> { static constexpr int value = CTATTN_I64; };
template <> struct DTypeCode<int16_t> { static constexpr int value = CTATTN_I16; };
template <> struct DTypeCode<int8_t> { static constexpr int value = CTATTN_I8; };
template <> struct DTypeCode<bool> { static constexpr int value = CTATTN_BOOL; };

// Type of the statistics the kernels keep beside a tensor of DType (row statistics, LSE,
// losses, optimizer moments): double for double, float for every narrower type.
template <typename DType> using StatOf = std::conditional_t<std::is_same_v<DType, double>, double, float>;

// Host-side element type of a DType buffer (std::vector<bool> packs bits, so bool tensors
// travel as bytes).
template <typename DType> using HostElem = std::conditional_t<std::is_same_v<DType, bool>, uint8_t, DType>;

template <typename V> constexpr bool kHalfLike = std::is_same_v<V, bf16> || std::is_same_v<V, f16>;

// Scalar conversions on the host: round to nearest even into bf16 / f16, truncation into
// integers, x != 0 into bool.
template <typename DType> inline DType fromFloat(float x) {
    if constexpr (std::is_same_v<DType, bf16>) return bf16::fromFloat(x);
    else if constexpr (std::is_same_v<DType, f16>) return f16::fromFloat(x);
    else if constexpr (std::is_same_v<DType, bool>) return x != 0.f;
    else return DType(x);
}
template <typename V> inline float toFloat(V x) {
    if constexpr (kHalfLike<V>) return x.toFloat();
    else return float(x);
}
// Scalars given or returned at full precision: exact for double (and integer) tensors,
// rounded once to the storage type otherwise.
template <typename DType> inline DType fromDouble(double x) {
    if constexpr (kHalfLike<DType> || std::is_same_v<DType, float>) return fromFloat<DType>(float(x));
    else if constexpr (std::is_same_v<DType, bool>) return x != 0.0;
    else return DType(x);
}
template <typename V> inline double toDouble(V x) {
    if constexpr (kHalfLike<V>) return double(x.toFloat());
    else return double(x);
}

// Caching device allocator for the host layer's buffers.  A freed block goes to a free list
// keyed by its rounded size and is handed out again to the next request of that size, with
// no HIP call.  Reuse is safe without events because every kernel and copy of the host layer
// is ordered on the one Runtime stream: work on a block's next owner is enqueued after all
// work on its previous owner.  hipMalloc runs only when no cached block fits (the first
// steps of a training loop); on hipErrorOutOfMemory the cache is returned to the driver and
// the allocation retried.  (hipFreeAsync on the default pool stalled the host for up to
// 10 ms per call in a training step.)
class BlockCache {
public:
    static BlockCache &instance() {
        static BlockCache *cache = new BlockCache();  // never destroyed: outlives static tensors
        return *cache;
    }

    void *allocate(size_t bytes) {
        const size_t size = rounded(bytes);
        {
            std::lock_guard<std::mutex> lock(mutex_);
            auto it = free_.find(size);
            if (it != free_.end() && !it->second.empty()) {
                void *p = it->second.back();
                it->second.pop_back();
                cachedBytes_ -= size;
                return p;
            }
        }
        void *p = nullptr;
        hipError_t e = hipMalloc(&p, size);
        if (e == hipErrorOutOfMemory) {
            (void)hipGetLastError();
            emptyCache();
            e = hipMalloc(&p, size);
        }
        hipCheck(e, "hipMalloc");
        std::lock_guard<std::mutex> lock(mutex_);
        reservedBytes_ += size;
        return p;
    }

    void release(void *p, size_t bytes) {
        std::lock_guard<std::mutex> lock(mutex_);
        free_[rounded(bytes)].push_back(p);
        cachedBytes_ += rounded(bytes);
    }

    // Returns every cached block to the driver (after the stream has drained).
    void emptyCache() {
        Runtime::synchronize();
        std::lock_guard<std::mutex> lock(mutex_);
        for (auto &[size, blocks] : free_) {
            for (void *p : blocks) (void)hipFree(p);
            reservedBytes_ -= size * blocks.size();
        }
        free_.clear();
        cachedBytes_ = 0;
    }

    size_t cachedBytes() {
        std::lock_guard<std::mutex> lock(mutex_);
        return cachedBytes_;
    }
    size_t reservedBytes() {
        std::lock_guard<std::mutex> lock(mutex_);
        return reservedBytes_;
    }

private:
    // 512-byte granules below 1 MiB, 64 KiB granules above.
    static size_t rounded(size_t bytes) {
        const size_t g = bytes < (size_t(1) << 20) ? 512 : (size_t(64) << 10);
        return (bytes + g - 1) / g * g;
    }

    std::mutex mutex_;
    std::map<size_t, std::vector<void *>> free_;
    size_t cachedBytes_ = 0, reservedBytes_ = 0;
};

// Device allocation from the block cache; the deleter hands the block back.
template <typename T>
std::shared_ptr<T[]> deviceAlloc(size_t count) {
    if (count == 0) return nullptr;
    const size_t bytes = count * sizeof(T);
    Runtime::stream();  // the stream (and device) exist before the first block
    void *p = BlockCache::instance().allocate(bytes);
    return std::shared_ptr<T[]>(static_cast<T *>(p), [bytes](T *q) { BlockCache::instance().release(q, bytes); });
}

template <typename DType = float>
class Tensor {
public:
    Tensor() = default;

    // Zero-initialised tensor of the given shape (Tensor.cu:36-43).
    explicit Tensor(const std::vector<size_t> &shape, float value = 0.f) : shape_(shape) {
        if (shape_.size() > 8) throw std::invalid_argument("Tensor does not support more than 8 dimensions");
        size_ = std::accumulate(shape_.begin(), shape_.end(), size_t(1), std::multiplies<size_t>());
        data_ = deviceAlloc<DType>(size_);
        version_ = std::make_shared<std::atomic<uint64_t>>(0);
        fill(value);
    }

    // Uninitialised tensor, for outputs a kernel overwrites completely.
    static Tensor empty(const std::vector<size_t> &shape) {
        Tensor t;
        if (shape.size() > 8) throw std::invalid_argument("Tensor does not support more than 8 dimensions");
        t.shape_ = shape;
        t.size_ = std::accumulate(shape.begin(), shape.end(), size_t(1), std::multiplies<size_t>());
        t.data_ = deviceAlloc<DType>(t.size_);
        t.version_ = std::make_shared<std::atomic<uint64_t>>(0);
        return t;
    }

    // Shallow wrap of an existing buffer (Tensor.cu:62-66).  The wrapper starts its own
    // version count (see version()).
    Tensor(std::shared_ptr<DType[]> data, const std::vector<size_t> &shape) : shape_(shape) {
        size_ = std::accumulate(shape_.begin(), shape_.end(), size_t(1), std::multiplies<size_t>());
        data_ = std::move(data);
        version_ = std::make_shared<std::atomic<uint64_t>>(0);
    }

    // Copies host values (in this DType's layout) into a new device tensor.
    static Tensor fromPointer(const std::vector<size_t> &shape, const DType *host) {
        Tensor t = empty(shape);
        if (t.size_ > 0) {
            hipCheck(hipMemcpyAsync(t.data_.get(), host, t.size_ * sizeof(DType), hipMemcpyHostToDevice,
                                    Runtime::stream()),
                     "hipMemcpyAsync H2D");
            Runtime::synchronize();  // `host` may be released as soon as we return
        }
        return t;
    }

    // Converts float host values to DType (round to nearest even for bf16) and uploads.
    static Tensor fromFloats(const std::vector<size_t> &shape, const float *host) {
        const size_t n = std::accumulate(shape.begin(), shape.end(), size_t(1), std::multiplies<size_t>());
        if constexpr (std::is_same_v<DType, float>) {
            return fromPointer(shape, host);
        } else {
            std::vector<HostElem<DType>> tmp(n);
            for (size_t i = 0; i < n; ++i) tmp[i] = HostElem<DType>(fromFloat<DType>(host[i]));
            return fromPointer(shape, reinterpret_cast<const DType *>(tmp.data()));
        }
    }

    // Device values on the host in their own type (waits for the stream).
    std::vector<HostElem<DType>> toHost() const {
        std::vector<HostElem<DType>> raw(size_);
        if (size_ > 0) {
            hipCheck(hipMemcpyAsync(raw.data(), data_.get(), size_ * sizeof(DType), hipMemcpyDeviceToHost,
                                    Runtime::stream()),
                     "hipMemcpyAsync D2H");
            Runtime::synchronize();
        }
        return raw;
    }

    // Device values as floats on the host (waits for the stream).
    std::vector<float> toFloats() const {
        std::vector<HostElem<DType>> raw = toHost();
        std::vector<float> out(size_);
        for (size_t i = 0; i < size_; ++i) out[i] = toFloat(raw[i]);
        return out;
    }

    // Deep copy (Tensor.cu:119-123, headers.cu:224-237), stream-ordered D2D.
    Tensor clone() const {
        Tensor t;
        t.shape_ = shape_;
        t.size_ = size_;
        t.data_ = deviceAlloc<DType>(size_);
        t.version_ = std::make_shared<std::atomic<uint64_t>>(0);
        if (size_ > 0)
            hipCheck(hipMemcpyAsync(t.data_.get(), data_.get(), size_ * sizeof(DType), hipMemcpyDeviceToDevice,
                                    Runtime::stream()),
                     "hipMemcpyAsync D2D");
        return t;
    }

    // Fills every element with `value` (Tensor.cu:360).  Zero is a stream-ordered memset;
    // other values are staged on the host.
    void fill(double value) {
        bumpVersion();
        if (size_ == 0) return;
        const DType v = fromDouble<DType>(value);
        uint8_t first;
        std::memcpy(&first, &v, 1);
        bool bytewise = true;
        for (size_t b = 0; b < sizeof(DType); ++b)
            bytewise = bytewise && reinterpret_cast<const uint8_t *>(&v)[b] == first;
        if (bytewise) {
            hipCheck(hipMemsetAsync(data_.get(), first, size_ * sizeof(DType), Runtime::stream()), "hipMemsetAsync");
        } else {
            std::vector<HostElem<DType>> tmp(size_, HostElem<DType>(v));
            hipCheck(hipMemcpyAsync(data_.get(), tmp.data(), size_ * sizeof(DType), hipMemcpyHostToDevice,
                                    Runtime::stream()),
                     "hipMemcpyAsync fill");
            Runtime::synchronize();
        }
    }

    // Shallow reshape (Tensor.cu:547-570).
    Tensor reshape(const std::vector<size_t> &shape) const {
        const size_t n = std::accumulate(shape.begin(), shape.end(), size_t(1), std::multiplies<size_t>());
        if (n != size_) throw std::invalid_argument("reshape: element count changes");
        Tensor t(data_, shape);
        t.version_ = version_;  // same buffer, same version count
        return t;
    }

    double item() const {
        if (size_ != 1) throw std::runtime_error("Tensor is not a scalar");
        return toDouble(toHost()[0]);
    }

    const std::vector<size_t> &shape() const { return shape_; }
    size_t shape(size_t dim) const {
        if (dim >= shape_.size()) throw std::invalid_argument("Invalid dimension");
        return shape_[dim];
    }
    size_t size() const { return size_; }
    size_t nDim() const { return shape_.size(); }
    DType *get() const { return data_.get(); }
    DType *data() {
        bumpVersion();  // a mutable view of the buffer: assume it is written
        return data_.get();
    }
    const DType *data() const { return data_.get(); }
    std::shared_ptr<DType[]> dataPtr() const { return data_; }
    bool empty() const { return data_ == nullptr; }

    // Count of in-place writes made through this tensor's API (fill, mutable data()), shared
    // by every shallow copy and reshape of it.  A cache that keeps a tensor by reference
    // records the count and treats a change as "contents changed" (FlashAttentionLayer's
    // cached output).  Kernel writes through get() are not counted.
    uint64_t version() const { return version_ ? version_->load() : 0; }
    void bumpVersion() {
        if (version_) version_->fetch_add(1);
    }

private:
    std::vector<size_t> shape_;
    size_t size_ = 0;
    std::shared_ptr<DType[]> data_;
    std::shared_ptr<std::atomic<uint64_t>> version_;
};

}  // namespace ct
