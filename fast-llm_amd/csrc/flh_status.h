// flh_status.h -- error codes and the per-thread last-error message shared by
// the kernel translation units and the C-ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include "../../include/fastllm_hip.h"

namespace flh {
// Records msg as this thread's last error and returns code.
int set_error(int code, const char * msg);
// 0 when e == hipSuccess, else records "<what>: <hip error string>" and
// returns FLH_ERR_HIP.
int hip_check(hipError_t e, const char * what);
// FLH_OK once flh_init has selected a device, else FLH_ERR_STATE.
int need_device();
}  // namespace flh
