// Compiled-kernel launcher of the spyre backend (torch.compile path).
//
// Reference: launchKernel (torch_spyre/csrc/module.cpp:64-170), which
// deserialises, patches, loads, compiles and runs a Spyre program on every
// call.  Here a kernel spec produced by the Inductor backend is parsed once
// and cached; each call is one or more launches of precompiled gfx950
// kernels.
#include <torch/extension.h>

#include "spyre_ops_common.h"

namespace spyre {

void launch_kernel(const std::string& spec, const std::vector<at::Tensor>& args) {
  TORCH_CHECK_NOT_IMPLEMENTED(false, "spyre: launch_kernel: kernel spec execution is not built yet");
}

}  // namespace spyre
