// lightllm::Tensor over HIP device memory (interface of the reference's
// include/lightllm/tensor.h:41-106).
#include "lightllm/tensor.h"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>
#include <stdexcept>

namespace lightllm {

namespace {
void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string("Tensor: ") + what + ": " + hipGetErrorString(e));
}
uint16_t f32_to_f16_bits(float x) {
    _Float16 h = (_Float16)x;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}
float f16_bits_to_f32(uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (float)h;
}
}  // namespace

Tensor::Tensor() = default;

Tensor::Tensor(std::vector<int> shape, DType dtype, Device device)
    : shape_(std::move(shape)), dtype_(dtype), device_(device), owns_data_(true) {
    for (int s : shape_)
        if (s < 0) throw std::runtime_error("Tensor: negative dimension");
    allocate();
}

Tensor::~Tensor() { deallocate(); }

Tensor::Tensor(Tensor&& o) noexcept
    : data_(o.data_), shape_(std::move(o.shape_)), dtype_(o.dtype_), device_(o.device_),
      owns_data_(o.owns_data_) {
    o.data_ = nullptr;
    o.owns_data_ = true;
}

Tensor& Tensor::operator=(Tensor&& o) noexcept {
    if (this != &o) {
        deallocate();
        data_ = o.data_;
        shape_ = std::move(o.shape_);
        dtype_ = o.dtype_;
        device_ = o.device_;
        owns_data_ = o.owns_data_;
        o.data_ = nullptr;
        o.owns_data_ = true;
    }
    return *this;
}

size_t Tensor::numel() const {
    if (shape_.empty()) return data_ ? 1 : 0;
    size_t n = 1;
    for (int s : shape_) n *= static_cast<size_t>(s);
    return n;
}

size_t Tensor::nbytes() const { return numel() * dtype_size(dtype_); }

void Tensor::allocate() {
    size_t bytes = nbytes();
    if (bytes == 0) return;
    if (device_ == Device::CUDA) {
        hip_check(hipMalloc(&data_, bytes), "hipMalloc");
    } else {
        data_ = std::malloc(bytes);
        if (!data_) throw std::runtime_error("Tensor: host allocation failed");
    }
}

void Tensor::deallocate() {
    if (data_ && owns_data_) {
        if (device_ == Device::CUDA) (void)hipFree(data_);
        else std::free(data_);
    }
    data_ = nullptr;
}

void Tensor::copy_from(const void* src, size_t bytes) {
    if (bytes > nbytes()) throw std::runtime_error("Tensor::copy_from: too many bytes");
    if (bytes == 0) return;
    if (device_ == Device::CUDA) hip_check(hipMemcpy(data_, src, bytes, hipMemcpyHostToDevice), "copy_from");
    else std::memcpy(data_, src, bytes);
}

void Tensor::copy_to(void* dst, size_t bytes) const {
    if (bytes > nbytes()) throw std::runtime_error("Tensor::copy_to: too many bytes");
    if (bytes == 0) return;
    if (device_ == Device::CUDA) hip_check(hipMemcpy(dst, data_, bytes, hipMemcpyDeviceToHost), "copy_to");
    else std::memcpy(dst, data_, bytes);
}

Tensor Tensor::view(std::vector<int> new_shape) const {
    Tensor t;
    t.shape_ = std::move(new_shape);
    t.dtype_ = dtype_;
    t.device_ = device_;
    t.owns_data_ = false;
    t.data_ = data_;
    if (t.numel() != numel()) {
        t.data_ = nullptr;
        throw std::runtime_error("Tensor::view: numel mismatch");
    }
    return t;
}

void Tensor::reshape_inplace(std::vector<int> new_shape) {
    size_t n = 1;
    for (int s : new_shape) n *= static_cast<size_t>(s);
    if (n != numel()) throw std::runtime_error("Tensor::reshape_inplace: numel mismatch");
    shape_ = std::move(new_shape);
}

void Tensor::fill_zeros() {
    if (!data_) return;
    if (device_ == Device::CUDA) hip_check(hipMemset(data_, 0, nbytes()), "fill_zeros");
    else std::memset(data_, 0, nbytes());
}

Tensor Tensor::wrap(void* data, std::vector<int> shape, DType dtype, Device device) {
    Tensor t;
    t.data_ = data;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.device_ = device;
    t.owns_data_ = false;
    return t;
}

std::string Tensor::to_string(int max_elems) const {
    std::ostringstream os;
    os << "Tensor(" << dtype_name(dtype_) << ", [";
    for (size_t i = 0; i < shape_.size(); ++i) os << (i ? "," : "") << shape_[i];
    os << "]) {";
    size_t n = std::min<size_t>(numel(), max_elems > 0 ? (size_t)max_elems : 0);
    std::vector<unsigned char> host(n * dtype_size(dtype_));
    if (n) copy_to(host.data(), host.size());
    for (size_t i = 0; i < n; ++i) {
        if (i) os << ", ";
        switch (dtype_) {
            case DType::F32: { float f; std::memcpy(&f, &host[i * 4], 4); os << f; break; }
            case DType::I32: { int v; std::memcpy(&v, &host[i * 4], 4); os << v; break; }
            case DType::F16: { uint16_t b; std::memcpy(&b, &host[i * 2], 2); os << f16_bits_to_f32(b); break; }
            case DType::BF16: {
                uint16_t b; std::memcpy(&b, &host[i * 2], 2);
                uint32_t u = (uint32_t)b << 16; float f; std::memcpy(&f, &u, 4); os << f; break;
            }
        }
    }
    if (numel() > n) os << ", ...";
    os << "}";
    (void)f32_to_f16_bits;
    return os.str();
}

}  // namespace lightllm
