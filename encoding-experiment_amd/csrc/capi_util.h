// Helpers shared by the extern "C" entry points: error translation, stream
// selection, host<->device staging.
#pragma once

#include <new>
#include <stdexcept>

#include "larql_hip_internal.h"

// Lock the context, make its device current, run `f`, and turn any failure into
// a negative status with a message in ctx->last_error.
template <class F>
static int guarded(larql_hip_ctx* c, F&& f) {
    if (!c) return LARQL_HIP_ERR_INVALID;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    try {
        LARQL_HIP_CHECK(hipSetDevice(c->device));
        f();
        c->last_error.clear();
        return LARQL_HIP_OK;
    } catch (const larql::Error& e) {
        c->last_error = e.msg;
        return e.code;
    } catch (const std::bad_alloc&) {
        c->last_error = "host allocation failed";
        return LARQL_HIP_ERR_NOMEM;
    } catch (const std::exception& e) {
        c->last_error = e.what();
        return LARQL_HIP_ERR_DEVICE;
    }
}

static inline hipStream_t pick_stream(larql_hip_ctx* c, void* s) {
    return s ? static_cast<hipStream_t>(s) : c->stream;
}

template <class T>
static T* stage_upload(larql_hip_ctx* c, larql::DeviceBuf& b, const T* host, size_t n) {
    T* d = static_cast<T*>(larql::ensure(c, b, n * sizeof(T)));
    LARQL_HIP_CHECK(hipMemcpyAsync(d, host, n * sizeof(T), hipMemcpyHostToDevice, c->stream));
    return d;
}

static inline void download(larql_hip_ctx* c, void* host, const void* dev, size_t bytes) {
    LARQL_HIP_CHECK(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, c->stream));
    LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));
}
