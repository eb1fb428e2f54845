#pragma once
/// lightllm::Tensor for the MI355X build -- the carrier type of the paged
/// KV-cache operator API.  Same interface as the reference's Tensor
/// (include/lightllm/tensor.h:14-106 of wjb554/lightllm): row-major, int
/// shape, F32/F16/BF16/I32, CPU or device ("CUDA" names the GPU device, kept
/// for source compatibility; memory is HIP device memory), move-only.

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace lightllm {

enum class DType : uint8_t { F32 = 0, F16 = 1, BF16 = 2, I32 = 3 };

enum class Device : uint8_t { CPU = 0, CUDA = 1 };

inline const char* dtype_name(DType dt) {
    switch (dt) {
        case DType::F32: return "f32";
        case DType::F16: return "f16";
        case DType::BF16: return "bf16";
        case DType::I32: return "i32";
    }
    return "unknown";
}

inline size_t dtype_size(DType dt) {
    switch (dt) {
        case DType::F32: return 4;
        case DType::F16: return 2;
        case DType::BF16: return 2;
        case DType::I32: return 4;
    }
    return 0;
}

class Tensor {
public:
    Tensor();
    Tensor(std::vector<int> shape, DType dtype, Device device);
    ~Tensor();

    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(Tensor&& other) noexcept;
    Tensor(const Tensor&) = delete;
    Tensor& operator=(const Tensor&) = delete;

    template <typename T>
    T* data() { return static_cast<T*>(data_); }
    template <typename T>
    const T* data() const { return static_cast<const T*>(data_); }

    void* raw() { return data_; }
    const void* raw() const { return data_; }

    /// Copy `bytes` from host memory into this tensor / from it to host memory.
    void copy_from(const void* src, size_t bytes);
    void copy_to(void* dst, size_t bytes) const;

    const std::vector<int>& shape() const { return shape_; }
    int dims() const { return static_cast<int>(shape_.size()); }
    int size(int dim) const { return shape_[(dim < 0) ? dims() + dim : dim]; }

    size_t numel() const;
    size_t nbytes() const;

    DType dtype() const { return dtype_; }
    Device device() const { return device_; }
    bool is_cpu() const { return device_ == Device::CPU; }
    bool is_cuda() const { return device_ == Device::CUDA; }
    bool defined() const { return data_ != nullptr; }

    /// Non-owning view with a new shape (same numel).
    Tensor view(std::vector<int> new_shape) const;
    /// Reshape in place (same numel).
    void reshape_inplace(std::vector<int> new_shape);

    void fill_zeros();
    std::string to_string(int max_elems = 16) const;

    /// Non-owning wrapper around existing memory (used by the C ABI shims).
    static Tensor wrap(void* data, std::vector<int> shape, DType dtype, Device device);

private:
    void* data_ = nullptr;
    std::vector<int> shape_;
    DType dtype_ = DType::F32;
    Device device_ = Device::CPU;
    bool owns_data_ = true;

    void allocate();
    void deallocate();
};

}  // namespace lightllm
