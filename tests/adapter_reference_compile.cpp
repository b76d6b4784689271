// Compile check (no link, no run): the C++ host adapter instantiated on the reference's own types
// -- GgufTensorView for the mapped-tensor calls, StorageRowView for the row dot, MappedGgufModel for
// the whole-model upload -- from the reference's headers (include/oracle/model/*.hpp).
#include "oracle/model/mapped_gguf.hpp"
#include "oracle/model/storage_decode.hpp"

#include "hip_quantized.hpp"

using oracle::backend::hip::QuantizedDevice;

template void QuantizedDevice::mapped_tensor_matvec<oracle::model::GgufTensorView>(
    const oracle::model::GgufTensorView&, std::span<const float>, std::span<float>);
template void QuantizedDevice::mapped_tensor_matmul<oracle::model::GgufTensorView>(
    const oracle::model::GgufTensorView&, std::size_t, std::span<const float>, std::span<float>);
template void QuantizedDevice::mapped_tensor_matmul_device<oracle::model::GgufTensorView>(
    const oracle::model::GgufTensorView&, std::size_t, const float*, float*);
template void QuantizedDevice::decode_mapped_tensor<oracle::model::GgufTensorView>(
    const oracle::model::GgufTensorView&, std::span<float>);
template float QuantizedDevice::storage_dot<oracle::model::StorageRowView>(const oracle::model::StorageRowView&,
                                                                           std::span<const float>);
template void QuantizedDevice::upload_model<oracle::model::MappedGgufModel>(const oracle::model::MappedGgufModel&);
