// tensor.h - owning (or borrowed) row-major tensor on the host or the GPU.
//
// Same public interface as the reference Tensor (include/firefly/tensor.h:15-85, src/tensor.cc:127-270):
// move-only, row-major strides, from_external() for non-owning views, clone(), reshape(), data()/shape()/
// strides()/dtype()/device()/numel()/nbytes()/is_view().  view<T, Rank>() returns a StridedView (the reference
// returns a std::mdspan, which this toolchain's C++ library does not ship) with the same call syntax:
// v(i, j, ...).
#pragma once

#include <array>
#include <cstdint>
#include <ostream>
#include <stdexcept>
#include <string>
#include <vector>

#include "firefly/types.h"

namespace firefly
{

template <typename T, size_t Rank>
class StridedView
{
public:
    StridedView(T* data, const std::array<int64_t, Rank>& extents, const std::array<int64_t, Rank>& strides)
        : data_(data), extents_(extents), strides_(strides)
    {
    }

    template <typename... I>
    T& operator()(I... idx) const
    {
        static_assert(sizeof...(I) == Rank, "StridedView: index count must equal the rank");
        const int64_t ix[] = {static_cast<int64_t>(idx)...};
        int64_t       off = 0;
        for (size_t r = 0; r < Rank; ++r) off += ix[r] * strides_[r];
        return data_[off];
    }

    int64_t extent(size_t r) const { return extents_[r]; }
    int64_t stride(size_t r) const { return strides_[r]; }
    T*      data_handle() const { return data_; }

private:
    T*                        data_;
    std::array<int64_t, Rank> extents_;
    std::array<int64_t, Rank> strides_;
};

class FIREFLY_API Tensor
{
public:
    Tensor() = default;
    Tensor(std::vector<int64_t> shape, DType dtype, Device device);
    ~Tensor();

    Tensor(const Tensor&) = delete;
    Tensor& operator=(const Tensor&) = delete;
    Tensor(Tensor&&) noexcept;
    Tensor& operator=(Tensor&&) noexcept;

    // Deep copy (synchronous for GPU tensors, like the reference's cudaMemcpy).
    Tensor clone() const;
    // Same element count, new row-major shape; throws std::runtime_error otherwise.
    void reshape(std::vector<int64_t> new_shape);
    void print() const;
    std::string to_string() const;
    friend FIREFLY_API std::ostream& operator<<(std::ostream& os, const Tensor& tensor);

    // Non-owning tensor over caller memory (row-major); the destructor does not free it.
    static Tensor from_external(void* data_ptr, std::vector<int64_t> shape, DType dtype, Device device);

    template <typename T, size_t Rank>
    StridedView<T, Rank> view() const
    {
        if (shape_.size() != Rank) throw std::runtime_error("Tensor rank mismatch in view()");
        std::array<int64_t, Rank> ext{}, str{};
        for (size_t r = 0; r < Rank; ++r)
        {
            ext[r] = shape_[r];
            str[r] = strides_[r];
        }
        return StridedView<T, Rank>(static_cast<T*>(data_ptr_), ext, str);
    }

    template <typename T>
    T* data_as() const
    {
        return static_cast<T*>(data_ptr_);
    }

    void*                       data() const { return data_ptr_; }
    const std::vector<int64_t>& shape() const { return shape_; }
    const std::vector<int64_t>& strides() const { return strides_; }
    DType                       dtype() const { return dtype_; }
    Device                      device() const { return device_; }
    int64_t                     numel() const { return numel_; }
    size_t                      nbytes() const { return static_cast<size_t>(numel_) * dtype_size(dtype_); }
    bool                        is_view() const { return is_view_; }

private:
    void release();
    void set_shape(std::vector<int64_t> shape);

    void*                data_ptr_ = nullptr;
    std::vector<int64_t> shape_;
    std::vector<int64_t> strides_;
    int64_t              numel_ = 0;
    DType                dtype_ = DType::F32;
    Device               device_ = Device::CPU;
    bool                 is_view_ = false;
};

}  // namespace firefly
