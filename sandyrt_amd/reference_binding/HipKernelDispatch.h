// HipKernelDispatch.h -- the reference-side binding of libsandyrt_hip (see
// HipKernelDispatch.cpp).  A SandyRT maintainer adds it to the reference tree
// as src/device/hip/HipKernelDispatch.h, beside the HipDevice that calls it.
#pragma once

#include "DeviceTypes.h"
#include "KernelIR.h"
#include "Result.h"
#include "Tensor.h"
#include "sandyrt_hip.h"

#include <cstdint>
#include <span>

namespace sandy::device {

// One operand of a launch, as HipDevice::run resolves it -- the fields of
// CudaDeviceBufferView (src/device/cuda/CudaKernels.h:19-28).  Dense: `data`
// is the allocation's device address and `view` its strides and storage
// offset.  Paged (the reference's CudaPagedTensor layout, inputs only): `data`
// is the device array of page start addresses, `view.desc` the logical shape,
// and growDim / pageSize / pageCount describe the pages.
struct HipDeviceBufferView {
    void* data = nullptr;
    TensorViewDesc view;
    bool paged = false;
    int64_t growDim = -1;
    int64_t pageSize = -1;
    int64_t pageCount = 0;
};

// Runs one KernelIR op on `stream` (a hipStream_t).  `inputs` / `outputs`
// follow the op's inputs() / outputs() order, as CudaDevice::run builds its
// CudaLaunchContext (src/device/cuda/CudaDevice.cpp:455-510).  Paged inputs
// of element-wise, reduction, gather, softmax, norm, RoPE and attention are
// read (attention K/V paged along the key dimension by the paged kernels,
// anything else gathered by sandy_hip_paged_stage); the other families
// reject them with the reference's wording; outputs must be dense.
Result<void> hip_run_kernel(const ir::kernel_ir::Op& op, std::span<const HipDeviceBufferView> inputs,
                            std::span<const HipDeviceBufferView> outputs, void* stream);

} // namespace sandy::device
