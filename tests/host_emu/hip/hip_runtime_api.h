// Host build of a HIP kernel source (test infrastructure): the few runtime
// types the C ABI header names.
#pragma once
typedef struct ihipStream_t* hipStream_t;
typedef struct ihipEvent_t* hipEvent_t;
typedef int hipError_t;
