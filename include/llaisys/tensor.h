/*
 * Tensor handle C-ABI. Every declaration is the reference's
 * include/llaisys/tensor.h:7-65 (same names, argument meaning and ownership:
 * tensorCreate/View/Permute/Slice return a new handle the caller frees with
 * tensorDestroy; views share storage).
 */
#ifndef LLAISYS_TENSOR_H
#define LLAISYS_TENSOR_H

#include "../llaisys.h"

__C {
    typedef struct LlaisysTensor *llaisysTensor_t;

    /* include/llaisys/tensor.h:9-14 */
    __export llaisysTensor_t tensorCreate(size_t *shape, size_t ndim, llaisysDataType_t dtype,
                                          llaisysDeviceType_t device_type, int device_id);
    /* :16-17 */
    __export void tensorDestroy(llaisysTensor_t tensor);
    /* :19-20 */
    __export void *tensorGetData(llaisysTensor_t tensor);
    /* :22-23 */
    __export size_t tensorGetNdim(llaisysTensor_t tensor);
    /* :25-27 */
    __export void tensorGetShape(llaisysTensor_t tensor, size_t *shape);
    /* :29-31 (strides in elements) */
    __export void tensorGetStrides(llaisysTensor_t tensor, ptrdiff_t *strides);
    /* :33-34 */
    __export llaisysDataType_t tensorGetDataType(llaisysTensor_t tensor);
    /* :36-37 */
    __export llaisysDeviceType_t tensorGetDeviceType(llaisysTensor_t tensor);
    /* :39-40 */
    __export int tensorGetDeviceId(llaisysTensor_t tensor);
    /* :42-43 */
    __export void tensorDebug(llaisysTensor_t tensor);
    /* :45-46 */
    __export uint8_t tensorIsContiguous(llaisysTensor_t tensor);
    /* :48-50: copy numel*elsize bytes of host memory into the tensor */
    __export void tensorLoad(llaisysTensor_t tensor, const void *data);
    /* :52-55 */
    __export llaisysTensor_t tensorView(llaisysTensor_t tensor, size_t *shape, size_t ndim);
    /* :57-59 */
    __export llaisysTensor_t tensorPermute(llaisysTensor_t tensor, size_t *order);
    /* :61-65: [start, end) along dim */
    __export llaisysTensor_t tensorSlice(llaisysTensor_t tensor, size_t dim, size_t start, size_t end);
}

#endif /* LLAISYS_TENSOR_H */
