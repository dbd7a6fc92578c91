// runtime.hip -- device / buffer / stream / event tier of libironmill_hip
// (counterpart of ironmill-metal-sys: device.rs, buffer.rs, command.rs).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <new>
#include <algorithm>
#include <string>

#include "imh_internal.h"

namespace imh {

static thread_local std::string g_last_error = "";

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return e == hipErrorOutOfMemory ? IMH_ENOMEM : IMH_EDEVICE;
}

void clear_error() { g_last_error.clear(); }

int use_device(const imh_device *dev) {
    int cur = -1;
    IMH_HIP(hipGetDevice(&cur));
    if (cur != dev->ordinal) IMH_HIP(hipSetDevice(dev->ordinal));
    return IMH_OK;
}

int stream_scratch(imh_stream *s, int slot, size_t bytes, void **out) {
    if (slot < 0 || slot >= kScratchSlots) return fail(IMH_EINVAL, "stream_scratch: bad slot");
    if (s->scratch_bytes[slot] < bytes) {
        if (s->capturing)
            return fail(IMH_EINVAL, "scratch memory must grow during stream capture: run the op once "
                                    "with the same shapes before capturing it");
        int rc = use_device(s->dev);
        if (rc) return rc;
        // grow by at least 2x so a run of growing shapes retires few blocks
        size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
        if (want < 2 * s->scratch_bytes[slot]) want = 2 * s->scratch_bytes[slot];
        void *fresh = nullptr;
        IMH_HIP(hipMalloc(&fresh, want));
        // the old block may be addressed by a captured graph: keep it until
        // the stream is freed (never free memory a replay could touch)
        if (s->scratch[slot]) {
            try {
                s->retired.push_back(s->scratch[slot]);
            } catch (...) {
                (void)hipFree(fresh);
                return fail(IMH_ENOMEM, "stream_scratch: host allocation failed");
            }
        }
        s->scratch[slot] = fresh;
        s->scratch_bytes[slot] = want;
    }
    *out = s->scratch[slot];
    return IMH_OK;
}

}  // namespace imh

// Byte fill used by imh_fill_zero: 16-byte stores for the aligned body.
__global__ void imh_fill_zero_kernel(uint8_t *dst, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t head = (16 - ((uintptr_t)dst & 15)) & 15;
    if (head > n) head = n;
    for (size_t j = i; j < head; j += stride) dst[j] = 0;
    uint4 *body = reinterpret_cast<uint4 *>(dst + head);
    size_t nv = (n - head) / 16;
    for (size_t j = i; j < nv; j += stride) body[j] = make_uint4(0, 0, 0, 0);
    for (size_t j = head + nv * 16 + i; j < n; j += stride) dst[j] = 0;
}

extern "C" {

const char *imh_last_error(void) { return imh::g_last_error.c_str(); }

int imh_device_count(int *count) {
    if (!count) return imh::fail(IMH_EINVAL, "imh_device_count: count is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        return imh::hip_fail(e, "hipGetDeviceCount");
    }
    *count = n;
    return IMH_OK;
}

int imh_device_open(int ordinal, imh_device **out) {
    if (!out) return imh::fail(IMH_EINVAL, "imh_device_open: out is NULL");
    *out = nullptr;
    int n = 0;
    IMH_HIP(hipGetDeviceCount(&n));
    if (ordinal < 0 || ordinal >= n)
        return imh::fail(IMH_EINVAL, "imh_device_open: ordinal " + std::to_string(ordinal) +
                                         " out of range (" + std::to_string(n) + " devices)");
    imh_device *d = new (std::nothrow) imh_device();
    if (!d) return imh::fail(IMH_ENOMEM, "imh_device_open: host allocation failed");
    d->ordinal = ordinal;
    hipError_t e = hipGetDeviceProperties(&d->props, ordinal);
    if (e != hipSuccess) {
        delete d;
        return imh::hip_fail(e, "hipGetDeviceProperties");
    }
    if (std::strncmp(d->props.gcnArchName, "gfx950", 6) != 0) {
        std::string arch = d->props.gcnArchName;
        delete d;
        return imh::fail(IMH_EUNSUPPORTED,
                         "imh_device_open: kernels are built for gfx950, device is " + arch);
    }
    // per-device set-up: the no-alloc attention's fixed scratch address
    int rc = imh::noalloc_scratch_init(ordinal);
    if (rc) {
        delete d;
        return rc;
    }
    *out = d;
    return IMH_OK;
}

void imh_device_free(imh_device *dev) { delete dev; }

int imh_device_get_info(const imh_device *dev, imh_device_info *out) {
    if (!dev || !out) return imh::fail(IMH_EINVAL, "imh_device_get_info: NULL argument");
    out->ordinal = dev->ordinal;
    out->compute_units = dev->props.multiProcessorCount;
    out->wavefront_size = dev->props.warpSize;
    out->clock_khz = dev->props.clockRate;
    out->total_global_mem = dev->props.totalGlobalMem;
    out->lds_per_block = dev->props.sharedMemPerBlock;
    std::snprintf(out->arch, sizeof(out->arch), "%s", dev->props.gcnArchName);
    return IMH_OK;
}

int imh_buffer_alloc(imh_device *dev, size_t length, imh_buffer **out) {
    if (!dev || !out) return imh::fail(IMH_EINVAL, "imh_buffer_alloc: NULL argument");
    *out = nullptr;
    if (length == 0) return imh::fail(IMH_EINVAL, "imh_buffer_alloc: zero length");
    int rc = imh::use_device(dev);
    if (rc) return rc;
    void *p = nullptr;
    IMH_HIP(hipMalloc(&p, length));
    imh_buffer *b = new (std::nothrow) imh_buffer{dev, p, length};
    if (!b) {
        (void)hipFree(p);
        return imh::fail(IMH_ENOMEM, "imh_buffer_alloc: host allocation failed");
    }
    *out = b;
    return IMH_OK;
}

int imh_buffer_alloc_with_data(imh_device *dev, const void *data, size_t length,
                               imh_buffer **out) {
    if (!data) return imh::fail(IMH_EINVAL, "imh_buffer_alloc_with_data: data is NULL");
    int rc = imh_buffer_alloc(dev, length, out);
    if (rc) return rc;
    rc = imh_buffer_write(*out, 0, data, length);
    if (rc) {
        imh_buffer_free(*out);
        *out = nullptr;
    }
    return rc;
}

void imh_buffer_free(imh_buffer *buf) {
    if (!buf) return;
    if (buf->ptr) {
        imh::use_device(buf->dev);
        (void)hipFree(buf->ptr);
    }
    delete buf;
}

size_t imh_buffer_length(const imh_buffer *buf) { return buf ? buf->length : 0; }

void *imh_buffer_device_ptr(const imh_buffer *buf) { return buf ? buf->ptr : nullptr; }

int imh_buffer_write(imh_buffer *buf, size_t offset, const void *src, size_t length) {
    if (!buf || (!src && length)) return imh::fail(IMH_EINVAL, "imh_buffer_write: NULL argument");
    if (offset > buf->length || length > buf->length - offset)
        return imh::fail(IMH_EINVAL, "imh_buffer_write: range [" + std::to_string(offset) + ", +" +
                                         std::to_string(length) + ") exceeds buffer of " +
                                         std::to_string(buf->length) + " bytes");
    if (!length) return IMH_OK;
    int rc = imh::use_device(buf->dev);
    if (rc) return rc;
    IMH_HIP(hipMemcpy(static_cast<uint8_t *>(buf->ptr) + offset, src, length,
                      hipMemcpyHostToDevice));
    return IMH_OK;
}

int imh_buffer_read(const imh_buffer *buf, size_t offset, void *dst, size_t length) {
    if (!buf || (!dst && length)) return imh::fail(IMH_EINVAL, "imh_buffer_read: NULL argument");
    if (offset > buf->length || length > buf->length - offset)
        return imh::fail(IMH_EINVAL, "imh_buffer_read: range [" + std::to_string(offset) + ", +" +
                                         std::to_string(length) + ") exceeds buffer of " +
                                         std::to_string(buf->length) + " bytes");
    if (!length) return IMH_OK;
    int rc = imh::use_device(buf->dev);
    if (rc) return rc;
    IMH_HIP(hipMemcpy(dst, static_cast<const uint8_t *>(buf->ptr) + offset, length,
                      hipMemcpyDeviceToHost));
    return IMH_OK;
}

int imh_copy_to_host(imh_device *dev, void *dst, const void *src, size_t length) {
    if (!dev || ((!dst || !src) && length)) return imh::fail(IMH_EINVAL, "imh_copy_to_host: NULL argument");
    if (!length) return IMH_OK;
    int rc = imh::use_device(dev);
    if (rc) return rc;
    IMH_HIP(hipMemcpy(dst, src, length, hipMemcpyDeviceToHost));
    return IMH_OK;
}

int imh_stream_create(imh_device *dev, imh_stream **out) {
    if (!dev || !out) return imh::fail(IMH_EINVAL, "imh_stream_create: NULL argument");
    *out = nullptr;
    int rc = imh::use_device(dev);
    if (rc) return rc;
    hipStream_t s;
    IMH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    imh_stream *st = new (std::nothrow) imh_stream{dev, s, {}, {}, false, {}};
    if (!st) {
        (void)hipStreamDestroy(s);
        return imh::fail(IMH_ENOMEM, "imh_stream_create: host allocation failed");
    }
    *out = st;
    return IMH_OK;
}

void imh_stream_free(imh_stream *stream) {
    if (!stream) return;
    imh::use_device(stream->dev);
    (void)hipStreamSynchronize(stream->stream);
    for (int i = 0; i < kScratchSlots; i++)
        if (stream->scratch[i]) (void)hipFree(stream->scratch[i]);
    for (void *p : stream->retired) (void)hipFree(p);
    (void)hipStreamDestroy(stream->stream);
    delete stream;
}

int imh_stream_sync(imh_stream *stream) {
    if (!stream) return imh::fail(IMH_EINVAL, "imh_stream_sync: NULL stream");
    IMH_HIP(hipStreamSynchronize(stream->stream));
    return IMH_OK;
}

void *imh_stream_native(imh_stream *stream) { return stream ? (void *)stream->stream : nullptr; }

int imh_fill_zero(imh_stream *stream, void *dst, size_t length) {
    if (!stream || (!dst && length)) return imh::fail(IMH_EINVAL, "imh_fill_zero: NULL argument");
    if (!length) return IMH_OK;
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    size_t blocks = (length / 16 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(imh_fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, stream->stream,
                       static_cast<uint8_t *>(dst), length);
    IMH_HIP(hipGetLastError());
    return IMH_OK;
}

int imh_stream_begin_capture(imh_stream *stream) {
    if (!stream) return imh::fail(IMH_EINVAL, "imh_stream_begin_capture: NULL stream");
    if (stream->capturing) return imh::fail(IMH_EINVAL, "imh_stream_begin_capture: already capturing");
    int rc = imh::use_device(stream->dev);
    if (rc) return rc;
    IMH_HIP(hipStreamBeginCapture(stream->stream, hipStreamCaptureModeThreadLocal));
    stream->capturing = true;
    return IMH_OK;
}

int imh_stream_end_capture(imh_stream *stream, imh_graph **out) {
    if (!stream || !out) return imh::fail(IMH_EINVAL, "imh_stream_end_capture: NULL argument");
    *out = nullptr;
    if (!stream->capturing) return imh::fail(IMH_EINVAL, "imh_stream_end_capture: stream is not capturing");
    stream->capturing = false;
    hipGraph_t g = nullptr;
    IMH_HIP(hipStreamEndCapture(stream->stream, &g));
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return imh::hip_fail(e, "hipGraphInstantiate");
    }
    imh_graph *gr = new (std::nothrow) imh_graph{stream->dev, g, ex, stream};
    if (!gr) {
        (void)hipGraphExecDestroy(ex);
        (void)hipGraphDestroy(g);
        return imh::fail(IMH_ENOMEM, "imh_stream_end_capture: host allocation failed");
    }
    *out = gr;
    return IMH_OK;
}

int imh_graph_launch(imh_graph *graph, imh_stream *stream) {
    if (!graph || !stream) return imh::fail(IMH_EINVAL, "imh_graph_launch: NULL argument");
    if (stream != graph->stream)
        return imh::fail(IMH_EINVAL, "imh_graph_launch: a graph replays on the stream it was captured on "
                                     "(its kernels use that stream's scratch memory)");
    if (stream->capturing) return imh::fail(IMH_EINVAL, "imh_graph_launch: the stream is capturing");
    IMH_HIP(hipGraphLaunch(graph->exec, stream->stream));
    return IMH_OK;
}

void imh_graph_free(imh_graph *graph) {
    if (!graph) return;
    (void)hipGraphExecDestroy(graph->exec);
    (void)hipGraphDestroy(graph->graph);
    delete graph;
}

int imh_event_create(imh_device *dev, imh_event **out) {
    if (!dev || !out) return imh::fail(IMH_EINVAL, "imh_event_create: NULL argument");
    *out = nullptr;
    int rc = imh::use_device(dev);
    if (rc) return rc;
    hipEvent_t e;
    IMH_HIP(hipEventCreate(&e));
    imh_event *ev = new (std::nothrow) imh_event{dev, e};
    if (!ev) {
        (void)hipEventDestroy(e);
        return imh::fail(IMH_ENOMEM, "imh_event_create: host allocation failed");
    }
    *out = ev;
    return IMH_OK;
}

void imh_event_free(imh_event *ev) {
    if (!ev) return;
    (void)hipEventDestroy(ev->ev);
    delete ev;
}

int imh_event_record(imh_event *ev, imh_stream *stream) {
    if (!ev || !stream) return imh::fail(IMH_EINVAL, "imh_event_record: NULL argument");
    IMH_HIP(hipEventRecord(ev->ev, stream->stream));
    return IMH_OK;
}

int imh_event_elapsed_ms(imh_event *start, imh_event *end, float *ms) {
    if (!start || !end || !ms) return imh::fail(IMH_EINVAL, "imh_event_elapsed_ms: NULL argument");
    IMH_HIP(hipEventSynchronize(end->ev));
    IMH_HIP(hipEventElapsedTime(ms, start->ev, end->ev));
    return IMH_OK;
}

int imh_kv_positions_for(uint32_t seq_pos, uint32_t token_count, uint32_t window_size, uint32_t max_seq_len,
                         imh_kv_positions *out) {
    const char *who = "imh_kv_positions_for";
    if (!out) return imh::fail(IMH_EINVAL, std::string(who) + ": NULL output");
    if ((uint64_t)seq_pos + token_count > max_seq_len)
        return imh::fail(IMH_ERANGE, std::string(who) + ": seq_pos " + std::to_string(seq_pos) + " + token_count " +
                                         std::to_string(token_count) + " exceeds max_seq_len " +
                                         std::to_string(max_seq_len));
    const uint32_t stride = window_size ? window_size : max_seq_len;
    if (token_count == 0 || token_count > stride)
        return imh::fail(IMH_EINVAL, std::string(who) + ": token_count must be 1..stride");
    out->stride = stride;
    if (window_size) {
        out->write_pos = seq_pos % window_size;
        const uint32_t effective = std::min<uint64_t>((uint64_t)seq_pos + token_count, window_size);
        out->attn_base = std::min(effective - token_count, stride - token_count);   // effective >= token_count
    } else {
        out->write_pos = seq_pos;
        out->attn_base = seq_pos;
    }
    out->attn_len = out->attn_base + token_count;
    return IMH_OK;
}

}  // extern "C"
