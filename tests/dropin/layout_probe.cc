// layout_probe.cc -- prints the layout facts that the reference's code and
// this library must agree on when one is linked against the other: sizes
// and alignments of the types whose members inline header code reads, the
// offsets of the CudaModelWeights counters the device runtime writes, and
// the enumerator values.  The drop-in Makefile builds it twice, against the
// reference's headers and against this library's stand-ins, and the
// drop-in test compares the two outputs line for line.
#include "include/cuda_kvcache.h"
#include "include/cuda_runtime.h"
#include "include/cuda_tensor.h"
#include "include/model.h"
#include "include/quantized_tensor.h"
#include "include/tensor.h"

#include <cstddef>
#include <cstdio>

using namespace yan_lamma;

#define TYPE(T) std::printf("%s size=%zu align=%zu\n", #T, sizeof(T), alignof(T))
#define FIELD(T, f) std::printf("%s.%s offset=%zu\n", #T, #f, offsetof(T, f))

int main() {
    TYPE(Tensor);
    TYPE(CudaDeviceBuffer);
    TYPE(CudaTensor);
    TYPE(CudaCache);
    TYPE(CudaAllocationStats);
    TYPE(CudaloadWeight);
    TYPE(CudaModelWeights);
    TYPE(Block_Q80);
    TYPE(Block_Q40);
    TYPE(Block_Q41);
    FIELD(CudaModelWeights, device_id);
    FIELD(CudaModelWeights, host_to_device_copies);
    FIELD(CudaModelWeights, device_to_host_copies);
    FIELD(CudaModelWeights, host_to_device_bytes);
    FIELD(CudaModelWeights, device_to_host_bytes);
    FIELD(CudaModelWeights, weights);
    FIELD(CudaloadWeight, buffer);
    std::printf("RopeType %d %d\n", int(kNormal), int(kNeoX));
    std::printf("QuantType %d %d %d %d %d\n", int(QuantType::kF32), int(QuantType::kF16),
                int(QuantType::kQ80), int(QuantType::kQ40), int(QuantType::kQ41));
    return 0;
}
