// HIP error check and graph-capture helper with the semantics of the
// reference's include/gpu_utils.hpp:7-14 (print and exit on a failed HIP call)
// and :45-59 (the single capture dependency of a stream is the node just
// enqueued; anything else throws).  The rocBLAS handle of the reference belongs
// to its GEMM path and is not part of this library.  Uses <cstdio> instead of
// <print> (not available in this toolchain's libstdc++).
//
// HIP_CHECK and last_captured_node follow include/gpu_utils.hpp:7-14
// and :45-59 of
// MarcVivas/llm-inference, which is distributed under this notice:
//
//   MIT License
//
//   Copyright (c) 2026 MarcVivas
//
//   Permission is hereby granted, free of charge, to any person obtaining a copy
//   of this software and associated documentation files (the "Software"), to deal
//   in the Software without restriction, including without limitation the rights
//   to use, copy, modify, merge, publish, distribute, sublicense, and/or sell
//   copies of the Software, and to permit persons to whom the Software is
//   furnished to do so, subject to the following conditions:
//
//   The above copyright notice and this permission notice shall be included in all
//   copies or substantial portions of the Software.
//
//   THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND, EXPRESS OR
//   IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF MERCHANTABILITY,
//   FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN NO EVENT SHALL THE
//   AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM, DAMAGES OR OTHER
//   LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR OTHERWISE, ARISING FROM,
//   OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE USE OR OTHER DEALINGS IN THE
//   SOFTWARE.
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
