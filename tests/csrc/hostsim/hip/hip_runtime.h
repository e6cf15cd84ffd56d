// TEST INFRASTRUCTURE ONLY: a host-only stand-in for the HIP runtime API, so
// the library's host code (secure_infer_amd/csrc/si_api.cpp, si_host.cpp)
// builds with g++ under ThreadSanitizer / AddressSanitizer.  Streams are
// worker threads, events are generation counters, device memory is host
// memory and the library's kernels run as CPU tasks in stream order
// (tests/csrc/hostsim/hostsim.cpp).  Only the names the library uses are
// declared; nothing here is linked into the product library.
#pragma once

#include <stddef.h>
#include <stdint.h>

typedef enum hipError_t {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorNotReady = 600,
    hipErrorUnknown = 999,
} hipError_t;

typedef struct ihipStream_t* hipStream_t;
typedef struct ihipEvent_t* hipEvent_t;

typedef enum hipMemcpyKind {
    hipMemcpyHostToHost = 0,
    hipMemcpyHostToDevice = 1,
    hipMemcpyDeviceToHost = 2,
    hipMemcpyDeviceToDevice = 3,
    hipMemcpyDefault = 4,
} hipMemcpyKind;

typedef enum hipDeviceAttribute_t {
    hipDeviceAttributeMultiprocessorCount = 1,
    hipDeviceAttributeWallClockRate = 2
} hipDeviceAttribute_t;

#define hipStreamDefault 0u
#define hipStreamNonBlocking 1u
#define hipEventDefault 0u
#define hipEventDisableTiming 2u
#define hipHostMallocDefault 0u

struct uint4 {
    unsigned int x, y, z, w;
};
static inline uint4 make_uint4(unsigned int x, unsigned int y, unsigned int z, unsigned int w)
{
    uint4 v;
    v.x = x;
    v.y = y;
    v.z = z;
    v.w = w;
    return v;
}

struct dim3 {
    unsigned int x, y, z;
    dim3(unsigned int a = 1, unsigned int b = 1, unsigned int c = 1) : x(a), y(b), z(c) {}
};

hipError_t hipGetDevice(int* dev);
hipError_t hipSetDevice(int dev);
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int dev);
hipError_t hipDeviceSynchronize(void);
hipError_t hipGetLastError(void);

hipError_t hipMalloc(void** p, size_t n);
hipError_t hipFree(void* p);
hipError_t hipMallocAsync(void** p, size_t n, hipStream_t s);
hipError_t hipFreeAsync(void* p, hipStream_t s);
hipError_t hipHostMalloc(void** p, size_t n, unsigned int flags);
hipError_t hipHostFree(void* p);
hipError_t hipHostGetDevicePointer(void** dev, void* host, unsigned int flags);
hipError_t hipMemcpy(void* dst, const void* src, size_t n, hipMemcpyKind k);
hipError_t hipMemset(void* p, int v, size_t n);
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind k, hipStream_t s);
hipError_t hipMemcpy2DAsync(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t height,
                            hipMemcpyKind k, hipStream_t s);

hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned int flags);
hipError_t hipStreamDestroy(hipStream_t s);
hipError_t hipStreamSynchronize(hipStream_t s);
hipError_t hipStreamWaitEvent(hipStream_t s, hipEvent_t e, unsigned int flags);

hipError_t hipEventCreate(hipEvent_t* e);
hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned int flags);
hipError_t hipEventDestroy(hipEvent_t e);
hipError_t hipEventRecord(hipEvent_t e, hipStream_t s);
hipError_t hipEventSynchronize(hipEvent_t e);
hipError_t hipEventQuery(hipEvent_t e);
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b);

template <class T>
static inline hipError_t hipMalloc(T** p, size_t n)
{
    return hipMalloc(reinterpret_cast<void**>(p), n);
}
