// tensor.cpp - Tensor storage, moves, views, clone and reshape.
#include <hip/hip_runtime_api.h>

#include <cstring>
#include <iostream>
#include <sstream>

#include "firefly/mm/allocator.h"
#include "firefly/tensor.h"

namespace firefly
{

namespace
{

void* alloc_on(Device d, size_t bytes)
{
    return d == Device::CPU ? DeviceAllocator<Device::CPU>::allocate(bytes)
                            : DeviceAllocator<Device::GPU>::allocate(bytes);
}

void free_on(Device d, void* p)
{
    if (d == Device::CPU)
        DeviceAllocator<Device::CPU>::free(p);
    else
        DeviceAllocator<Device::GPU>::free(p);
}

}  // namespace

void Tensor::set_shape(std::vector<int64_t> shape)
{
    shape_ = std::move(shape);
    strides_.assign(shape_.size(), 1);
    int64_t s = 1;
    for (size_t i = shape_.size(); i-- > 0;)
    {
        strides_[i] = s;
        s *= shape_[i];
    }
}

Tensor::Tensor(std::vector<int64_t> shape, DType dtype, Device device) : dtype_(dtype), device_(device)
{
    set_shape(std::move(shape));
    numel_ = 1;  // an empty shape is a scalar, as in the reference (src/tensor.cc:141)
    for (int64_t d : shape_) numel_ *= d;
    const size_t bytes = nbytes();
    if (bytes > 0) data_ptr_ = alloc_on(device_, bytes);
}

void Tensor::release()
{
    if (data_ptr_ != nullptr && !is_view_) free_on(device_, data_ptr_);
    data_ptr_ = nullptr;
}

Tensor::~Tensor() { release(); }

Tensor::Tensor(Tensor&& o) noexcept
    : data_ptr_(o.data_ptr_),
      shape_(std::move(o.shape_)),
      strides_(std::move(o.strides_)),
      numel_(o.numel_),
      dtype_(o.dtype_),
      device_(o.device_),
      is_view_(o.is_view_)
{
    o.data_ptr_ = nullptr;
    o.numel_ = 0;
}

Tensor& Tensor::operator=(Tensor&& o) noexcept
{
    if (this != &o)
    {
        release();
        data_ptr_ = o.data_ptr_;
        shape_ = std::move(o.shape_);
        strides_ = std::move(o.strides_);
        numel_ = o.numel_;
        dtype_ = o.dtype_;
        device_ = o.device_;
        is_view_ = o.is_view_;
        o.data_ptr_ = nullptr;
        o.numel_ = 0;
    }
    return *this;
}

Tensor Tensor::from_external(void* data_ptr, std::vector<int64_t> shape, DType dtype, Device device)
{
    Tensor t;
    t.data_ptr_ = data_ptr;
    t.dtype_ = dtype;
    t.device_ = device;
    t.is_view_ = true;
    t.set_shape(std::move(shape));
    t.numel_ = 0;  // an empty shape describes no elements here (src/tensor.cc:205-208)
    if (!t.shape_.empty())
    {
        t.numel_ = 1;
        for (int64_t d : t.shape_) t.numel_ *= d;
    }
    return t;
}

Tensor Tensor::clone() const
{
    Tensor       c(shape_, dtype_, device_);
    const size_t bytes = nbytes();
    if (bytes == 0 || data_ptr_ == nullptr) return c;
    if (device_ == Device::CPU)
    {
        std::memcpy(c.data_ptr_, data_ptr_, bytes);
    }
    else
    {
        // stream-ordered allocation above: order the copy after it, then wait, like the reference's cudaMemcpy
        hipStream_t s = static_cast<hipStream_t>(DeviceAllocator<Device::GPU>::get_default_stream());
        if (hipMemcpyAsync(c.data_ptr_, data_ptr_, bytes, hipMemcpyDeviceToDevice, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess)
            throw std::runtime_error("Tensor clone failed: device copy error");
    }
    return c;
}

void Tensor::reshape(std::vector<int64_t> new_shape)
{
    int64_t n = 1;
    for (int64_t d : new_shape) n *= d;
    if (n != numel_) throw std::runtime_error("Reshape: numel mismatch");
    set_shape(std::move(new_shape));
}

std::string Tensor::to_string() const
{
    std::ostringstream os;
    os << "Tensor(shape=[";
    for (size_t i = 0; i < shape_.size(); ++i) os << (i ? ", " : "") << shape_[i];
    os << "], dtype=" << dtype_to_string(dtype_) << ", device=" << (device_ == Device::CPU ? "CPU" : "GPU")
       << (is_view_ ? ", view" : "") << ")";
    return os.str();
}

void Tensor::print() const { std::cout << to_string() << std::endl; }

std::ostream& operator<<(std::ostream& os, const Tensor& t) { return os << t.to_string(); }

}  // namespace firefly
