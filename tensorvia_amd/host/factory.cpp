// Device -> TensorImpl factory registry (reference src/factory.cpp:7-47).
#include <mutex>
#include <string>
#include <unordered_map>

#include "tensorvia/factory.h"

using namespace via;

namespace {
std::unordered_map<Device, TensorImplFactory>& factories() {
    static std::unordered_map<Device, TensorImplFactory> f;
    return f;
}
std::mutex& factories_mu() {
    static std::mutex m;
    return m;
}
TensorImplFactory find(Device device) {
    std::lock_guard<std::mutex> lk(factories_mu());
    auto it = factories().find(device);
    if (it == factories().end())
        throw std::runtime_error("No tensor implementation registered for device: " + std::string(device_to_string(device)));
    return it->second;
}
} // namespace

void register_tensor_impl(Device device, TensorImplFactory factory) {
    std::lock_guard<std::mutex> lk(factories_mu());
    factories()[device] = std::move(factory);
}

std::shared_ptr<TensorImpl> create_tensor_impl(size_t numel, DataType dtype, Device device) {
    if (numel == 0) throw std::invalid_argument("numel must be bigger than 0");
    return find(device)(nullptr, numel, dtype);
}

std::shared_ptr<TensorImpl> create_tensor_impl(void* ptr, size_t numel, DataType dtype, Device device) {
    if (ptr == nullptr) throw std::runtime_error("create_tensor_impl: ptr is null");
    if (numel == 0) throw std::invalid_argument("numel must be bigger than 0");
    return find(device)(ptr, numel, dtype);
}
