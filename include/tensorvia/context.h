// Backend context interface (reference include/core/context.h:3-7).
#pragma once

class ContextImpl {
public:
    virtual ~ContextImpl() = default;
    // Backend-specific handle (the HIP backend returns a pointer to its hipStream_t).
    virtual void* ctx_raw_ptr() = 0;
};
