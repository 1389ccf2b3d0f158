// hip_utils.h -- error checking and event timing for the cuinfer C++ layer.
//
// Same convention as the reference's CUINFER_CHECK_CUDA
// (ref:include/cuinfer/cuda_utils.h:12-20): a failing call throws
// std::runtime_error("HIP error at <file>:<line> -- <message>").
#pragma once

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>

#include "../cri.h"

namespace cuinfer {

#define CUINFER_CHECK_HIP(expr)                                                                   \
    do {                                                                                          \
        hipError_t err_ = (expr);                                                                 \
        if (err_ != hipSuccess) {                                                                 \
            throw std::runtime_error(std::string("HIP error at ") + __FILE__ + ":" +            \
                                     std::to_string(__LINE__) + " -- " + hipGetErrorString(err_)); \
        }                                                                                         \
    } while (0)

// Throws std::runtime_error carrying cri_last_error_string() when a C-ABI call fails.
#define CUINFER_CHECK_CRI(expr)                                                                   \
    do {                                                                                          \
        int st_ = (expr);                                                                         \
        if (st_ != CRI_OK) {                                                                      \
            throw std::runtime_error(std::string("cretif error ") + std::to_string(st_) + " at " + \
                                     __FILE__ + ":" + std::to_string(__LINE__) + " -- " +         \
                                     cri_last_error_string());                                    \
        }                                                                                         \
    } while (0)

// hipEvent timer, the counterpart of CudaTimer (ref:include/cuinfer/cuda_utils.h:79-113).
class HipTimer {
public:
    HipTimer() {
        CUINFER_CHECK_HIP(hipEventCreate(&start_));
        CUINFER_CHECK_HIP(hipEventCreate(&stop_));
    }
    ~HipTimer() {
        (void)hipEventDestroy(start_);
        (void)hipEventDestroy(stop_);
    }
    HipTimer(const HipTimer&) = delete;
    HipTimer& operator=(const HipTimer&) = delete;
    void start(hipStream_t stream = 0) { CUINFER_CHECK_HIP(hipEventRecord(start_, stream)); }
    void stop(hipStream_t stream = 0) {
        CUINFER_CHECK_HIP(hipEventRecord(stop_, stream));
        CUINFER_CHECK_HIP(hipEventSynchronize(stop_));
    }
    float elapsed_ms() const {
        float ms = 0.0f;
        CUINFER_CHECK_HIP(hipEventElapsedTime(&ms, start_, stop_));
        return ms;
    }

private:
    hipEvent_t start_{};
    hipEvent_t stop_{};
};

}  // namespace cuinfer
