// HIP error check and graph-capture helper with the semantics of the
// reference's include/gpu_utils.hpp:7-14 (print and exit on a failed HIP call)
// and :45-59 (the single capture dependency of a stream is the node just
// enqueued; anything else throws).  The rocBLAS handle of the reference belongs
// to its GEMM path and is not part of this library.  Uses <cstdio> instead of
// <print> (not available in this toolchain's libstdc++).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <stdexcept>

#define HIP_CHECK(command)                                                               \
    do {                                                                                 \
        hipError_t status = (command);                                                   \
        if (status != hipSuccess) {                                                      \
            std::fprintf(stderr, "[HIP Error] %s at %s:%d\n", hipGetErrorString(status),  \
                         __FILE__, __LINE__);                                            \
            std::exit(EXIT_FAILURE);                                                     \
        }                                                                                \
    } while (0)

inline hipGraphNode_t last_captured_node(hipStream_t stream) {
    hipStreamCaptureStatus capture_status;
    const hipGraphNode_t* dependencies = nullptr;
    size_t count = 0;
    HIP_CHECK(hipStreamGetCaptureInfo_v2(stream, &capture_status, nullptr, nullptr,
                                         &dependencies, &count));
    if (capture_status != hipStreamCaptureStatusActive || count != 1) {
        throw std::runtime_error("Expected one capture dependency");
    }
    return dependencies[0];
}
