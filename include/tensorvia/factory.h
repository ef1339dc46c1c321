// Device -> TensorImpl factory registry (reference include/core/factory.h:10-18, src/factory.cpp).
#pragma once

#include <functional>
#include <memory>

#include "tensor.h"

// ptr == nullptr: uninitialised storage of numel elements; otherwise a deep copy of numel elements
// from host memory at ptr (a host -> device copy for device backends).
using TensorImplFactory = std::function<std::shared_ptr<TensorImpl>(void* ptr, size_t numel, via::DataType)>;

void register_tensor_impl(via::Device device, TensorImplFactory factory);

std::shared_ptr<TensorImpl> create_tensor_impl(size_t numel, via::DataType dtype, via::Device device);
std::shared_ptr<TensorImpl> create_tensor_impl(void* ptr, size_t numel, via::DataType dtype, via::Device device);

// Whole-storage copies between the HIP device and host (one definition per build, as in the
// reference's per-backend copy files).
void copy_device_to_host(std::shared_ptr<TensorImpl> src, std::shared_ptr<TensorImpl> dst, via::DataType dtype);
void copy_host_to_device(std::shared_ptr<TensorImpl> src, std::shared_ptr<TensorImpl> dst, via::DataType dtype);
