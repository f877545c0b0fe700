// Device runtime of libl0hip: the counterpart of LevelZero.LevelZeroRuntime,
// ComputeDevice and SharedBuffer<T> as the reference uses them
// (LevelZeroLlmEngine.cs:351-370, LlmModel.cs:353-443, LlmSequenceState.cs:60-79).
//
// One HIP stream per device carries every operation in order. Recording
// (BeginRecording/EndRecording, one command list per token in the reference)
// becomes HIP stream capture into a graph that is launched and waited for at
// l0h_end_recording; the executable graph is kept and updated in place with
// hipGraphExecUpdate when the next recording has the same topology.
#include "common.h"

#include <algorithm>
#include <cstring>

namespace l0h {

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(L0H_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
    return L0H_OK;
}

int use_device(l0h_device* dev) {
    if (!dev) return fail(L0H_ERR_INVALID_ARG, "device is null");
    L0H_HIP_TRY(hipSetDevice(dev->ordinal));
    return L0H_OK;
}

__global__ void zero_words_kernel(uint32_t* p, size_t words) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < words; i += stride) p[i] = 0u;
}

__global__ void zero_bytes_kernel(uint8_t* p, size_t bytes) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < bytes) p[i] = 0;
}

// Streaming read of n16 16-byte chunks (non-temporal loads, 8 per thread in flight, grid-stride):
// the read rate a weight-streaming kernel can reach on this device. The XOR keeps the loads live.
__global__ __launch_bounds__(256) void read_stream_kernel(const uint4* p, size_t n16, unsigned* sink) {
    constexpr int U = 8;
    const size_t nth = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    unsigned acc = 0;
    for (; i + (U - 1) * nth < n16; i += U * nth) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = ld_nt16(p + i + u * nth);
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += nth) {
        const uint4 v = ld_nt16(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;  // practically never: only so the loads are not removed
}

// Zero fill by kernel (not hipMemsetAsync), so it is safe inside a captured graph.
static int zero_fill(hipStream_t s, void* p, size_t bytes) {
    if (bytes == 0) return L0H_OK;
    uintptr_t addr = (uintptr_t)p;
    if ((addr & 3) == 0 && (bytes & 3) == 0) {
        size_t words = bytes / 4;
        unsigned blocks = (unsigned)std::min<size_t>(ceil_div(words, 256), 4096);
        zero_words_kernel<<<blocks, 256, 0, s>>>(static_cast<uint32_t*>(p), words);
    } else {
        zero_bytes_kernel<<<ceil_div(bytes, 256), 256, 0, s>>>(static_cast<uint8_t*>(p), bytes);
    }
    return launch_status("zero fill");
}

void drop_recording(l0h_device* dev) {
    if (!dev->cached_exec) return;
    (void)hipGraphExecDestroy(dev->cached_exec);
    dev->cached_exec = nullptr;
    dev->recording_dropped = true;
}

int ensure_workspace(l0h_device* dev, size_t bytes, size_t tickets) {
    if (bytes > dev->workspace_bytes) {
        if (dev->recording)
            return fail(L0H_ERR_INVALID_OP,
                        "split-reduction workspace must be sized before recording starts");
        L0H_HIP_TRY(hipStreamSynchronize(dev->stream));
        drop_recording(dev);  // the kept graph may address the old workspace
        if (dev->workspace) L0H_HIP_TRY(hipFree(dev->workspace));
        dev->workspace = nullptr;
        dev->workspace_bytes = 0;
        size_t want = std::max<size_t>(bytes, 1 << 20);
        L0H_HIP_TRY(hipMalloc(&dev->workspace, want));
        dev->workspace_bytes = want;
    }
    if (tickets > dev->ticket_count) {
        if (dev->recording)
            return fail(L0H_ERR_INVALID_OP, "completion counters must be sized before recording starts");
        L0H_HIP_TRY(hipStreamSynchronize(dev->stream));
        drop_recording(dev);
        if (dev->tickets) L0H_HIP_TRY(hipFree(dev->tickets));
        dev->tickets = nullptr;
        dev->ticket_count = 0;
        size_t want = std::max<size_t>(tickets, 4096);
        L0H_HIP_TRY(hipMalloc(&dev->tickets, want * sizeof(unsigned)));
        int st = zero_fill(dev->stream, dev->tickets, want * sizeof(unsigned));
        if (st) return st;
        L0H_HIP_TRY(hipStreamSynchronize(dev->stream));
        dev->ticket_count = want;
    }
    return L0H_OK;
}

}  // namespace l0h

using namespace l0h;

extern "C" {

int l0h_runtime_is_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return 0;
    }
    for (int i = 0; i < n; i++) {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, i) == hipSuccess && std::strncmp(p.gcnArchName, "gfx950", 6) == 0)
            return 1;
    }
    return 0;
}

int l0h_device_count(int* count) {
    L0H_CHECK_ARG(count, "count is null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        return fail(L0H_ERR_DEVICE, std::string("hipGetDeviceCount: ") + hipGetErrorString(e));
    }
    *count = n;
    return L0H_OK;
}

int l0h_device_open(int ordinal, l0h_device** out) {
    L0H_CHECK_ARG(out, "out is null");
    *out = nullptr;
    int n = 0;
    L0H_HIP_TRY(hipGetDeviceCount(&n));
    if (ordinal < 0 || ordinal >= n)
        return fail(L0H_ERR_INVALID_ARG, "device ordinal " + std::to_string(ordinal) + " out of range");
    L0H_HIP_TRY(hipSetDevice(ordinal));
    hipDeviceProp_t p;
    L0H_HIP_TRY(hipGetDeviceProperties(&p, ordinal));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(L0H_ERR_UNSUPPORTED, std::string("device is ") + p.gcnArchName + ", this library is built for gfx950");
    auto* d = new l0h_device();
    d->ordinal = ordinal;
    d->compute_units = p.multiProcessorCount;
    if (hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&d->upload, hipStreamNonBlocking) != hipSuccess) {
        delete d;
        return fail(L0H_ERR_DEVICE, "stream creation failed");
    }
    int st = ensure_workspace(d, 1 << 20, 4096);
    if (!st) st = static_scratch_init(d);  // hipSetDevice(ordinal) above: the device is current
    if (st) {
        l0h_device_close(d);
        return st;
    }
    clear_error();
    *out = d;
    return L0H_OK;
}

int l0h_device_close(l0h_device* dev) {
    if (!dev) return L0H_OK;
    (void)hipSetDevice(dev->ordinal);
    if (dev->recording) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(dev->stream, &g);
        if (g) (void)hipGraphDestroy(g);
    }
    if (dev->stream) (void)hipStreamSynchronize(dev->stream);
    if (dev->cached_exec) (void)hipGraphExecDestroy(dev->cached_exec);
    if (dev->workspace) (void)hipFree(dev->workspace);
    if (dev->tickets) (void)hipFree(dev->tickets);
    if (dev->q8_scratch) (void)hipFree(dev->q8_scratch);
    if (dev->stream) (void)hipStreamDestroy(dev->stream);
    if (dev->upload) (void)hipStreamDestroy(dev->upload);
    delete dev;
    return L0H_OK;
}

int l0h_device_info(l0h_device* dev, char* host_name, size_t name_bytes, int* compute_units) {
    int st = use_device(dev);
    if (st) return st;
    hipDeviceProp_t p;
    L0H_HIP_TRY(hipGetDeviceProperties(&p, dev->ordinal));
    if (host_name && name_bytes) {
        std::snprintf(host_name, name_bytes, "%s (%s)", p.name, p.gcnArchName);
    }
    if (compute_units) *compute_units = p.multiProcessorCount;
    return L0H_OK;
}

int l0h_alloc(l0h_device* dev, size_t bytes, void** out) {
    L0H_CHECK_ARG(out, "out is null");
    *out = nullptr;
    int st = use_device(dev);
    if (st) return st;
    if (dev->recording) return fail(L0H_ERR_INVALID_OP, "cannot allocate while recording");
    if (bytes == 0) bytes = 4;
    hipError_t e = hipMalloc(out, bytes);
    if (e != hipSuccess) {
        *out = nullptr;
        return fail(e == hipErrorOutOfMemory ? L0H_ERR_OUT_OF_MEMORY : L0H_ERR_DEVICE,
                    std::string("hipMalloc(") + std::to_string(bytes) + "): " + hipGetErrorString(e));
    }
    return L0H_OK;
}

int l0h_free(l0h_device* dev, void* ptr) {
    if (!ptr) return L0H_OK;
    int st = use_device(dev);
    if (st) return st;
    if (dev->recording) return fail(L0H_ERR_INVALID_OP, "cannot free while recording");
    L0H_HIP_TRY(hipStreamSynchronize(dev->stream));
    drop_recording(dev);  // the kept graph may address this buffer
    L0H_HIP_TRY(hipFree(ptr));
    return L0H_OK;
}

int l0h_write(l0h_device* dev, void* dst, size_t off, const void* host_src, size_t bytes) {
    int st = use_device(dev);
    if (st) return st;
    L0H_CHECK_ARG(dst && (host_src || bytes == 0), "null pointer");
    if (bytes == 0) return L0H_OK;
    char* d = static_cast<char*>(dst) + off;
    if (dev->recording) {
        // The reference writes shared memory at record time (LlmDecoderLayer.cs:320); the value
        // is read when the list executes. Same here: copied now, outside the captured stream.
        L0H_HIP_TRY(hipMemcpyAsync(d, host_src, bytes, hipMemcpyHostToDevice, dev->upload));
        L0H_HIP_TRY(hipStreamSynchronize(dev->upload));
    } else {
        L0H_HIP_TRY(hipMemcpyAsync(d, host_src, bytes, hipMemcpyHostToDevice, dev->stream));
        L0H_HIP_TRY(hipStreamSynchronize(dev->stream));
    }
    return L0H_OK;
}

int l0h_read(l0h_device* dev, const void* src, size_t off, void* host_dst, size_t bytes) {
    int st = use_device(dev);
    if (st) return st;
    L0H_CHECK_ARG(src && (host_dst || bytes == 0), "null pointer");
    if (dev->recording) return fail(L0H_ERR_INVALID_OP, "cannot read a buffer while recording");
    if (bytes == 0) return L0H_OK;
    L0H_HIP_TRY(hipMemcpyAsync(host_dst, static_cast<const char*>(src) + off, bytes,
                               hipMemcpyDeviceToHost, dev->stream));
    L0H_HIP_TRY(hipStreamSynchronize(dev->stream));
    return L0H_OK;
}

int l0h_fill_zero(l0h_device* dev, void* dst, size_t bytes) {
    int st = use_device(dev);
    if (st) return st;
    L0H_CHECK_ARG(dst || bytes == 0, "null pointer");
    return zero_fill(dev->stream, dst, bytes);
}

int l0h_begin_recording(l0h_device* dev) {
    int st = use_device(dev);
    if (st) return st;
    if (dev->recording) return fail(L0H_ERR_INVALID_OP, "already recording");
    L0H_HIP_TRY(hipStreamSynchronize(dev->stream));
    L0H_HIP_TRY(hipStreamBeginCapture(dev->stream, hipStreamCaptureModeRelaxed));
    dev->recording = true;
    return L0H_OK;
}

int l0h_end_recording(l0h_device* dev) {
    int st = use_device(dev);
    if (st) return st;
    if (!dev->recording) return fail(L0H_ERR_INVALID_OP, "not recording");
    dev->recording = false;
    hipGraph_t graph = nullptr;
    L0H_HIP_TRY(hipStreamEndCapture(dev->stream, &graph));
    size_t nodes = 0;
    dev->recorded_nodes = hipGraphGetNodes(graph, nullptr, &nodes) == hipSuccess ? (int)nodes : 0;
    bool reused = false;
    if (dev->cached_exec) {
        hipGraphNode_t err_node = nullptr;
        hipGraphExecUpdateResult res;
        if (hipGraphExecUpdate(dev->cached_exec, graph, &err_node, &res) == hipSuccess &&
            res == hipGraphExecUpdateSuccess) {
            reused = true;
        } else {
            (void)hipGetLastError();
            (void)hipGraphExecDestroy(dev->cached_exec);
            dev->cached_exec = nullptr;
        }
    }
    if (!reused) {
        hipError_t e = hipGraphInstantiate(&dev->cached_exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            dev->cached_exec = nullptr;
            (void)hipGraphDestroy(graph);
            return fail(L0H_ERR_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
        }
    }
    dev->recording_dropped = false;
    hipError_t e = hipGraphLaunch(dev->cached_exec, dev->stream);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("hipGraphLaunch: ") + hipGetErrorString(e));
    L0H_HIP_TRY(hipStreamSynchronize(dev->stream));
    return L0H_OK;
}

int l0h_recording_launches(l0h_device* dev, int* launches) {
    L0H_CHECK_ARG(dev && launches, "null argument");
    *launches = dev->recorded_nodes;
    return L0H_OK;
}

int l0h_replay_recording(l0h_device* dev, int count, float* ms_per_replay) {
    int st = use_device(dev);
    if (st) return st;
    L0H_CHECK_ARG(count > 0 && ms_per_replay, "count must be positive and ms_per_replay non-null");
    if (dev->recording) return fail(L0H_ERR_INVALID_OP, "the device is recording");
    if (!dev->cached_exec)
        return fail(L0H_ERR_INVALID_OP, dev->recording_dropped
                                            ? "memory used by the last recording was freed or moved since; record again"
                                            : "nothing has been recorded");
    hipEvent_t a = nullptr, b = nullptr;
    L0H_HIP_TRY(hipEventCreate(&a));
    hipError_t e = hipEventCreate(&b);
    if (e == hipSuccess) e = hipEventRecord(a, dev->stream);
    for (int i = 0; i < count && e == hipSuccess; i++) e = hipGraphLaunch(dev->cached_exec, dev->stream);
    if (e == hipSuccess) e = hipEventRecord(b, dev->stream);
    if (e == hipSuccess) e = hipEventSynchronize(b);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
    (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (e != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("replay: ") + hipGetErrorString(e));
    *ms_per_replay = ms / (float)count;
    return L0H_OK;
}

int l0h_abort_recording(l0h_device* dev) {
    int st = use_device(dev);
    if (st) return st;
    if (!dev->recording) return L0H_OK;
    dev->recording = false;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(dev->stream, &graph);
    if (graph) (void)hipGraphDestroy(graph);
    if (e != hipSuccess) {
        (void)hipGetLastError();
    }
    return L0H_OK;
}

int l0h_is_recording(l0h_device* dev, int* out) {
    L0H_CHECK_ARG(dev && out, "null pointer");
    *out = dev->recording ? 1 : 0;
    return L0H_OK;
}

int l0h_device_read_bandwidth(l0h_device* dev, size_t bytes, int reps, double* gbs) {
    int st = use_device(dev);
    if (st) return st;
    L0H_CHECK_ARG(gbs && reps > 0 && bytes >= (1u << 20), "need gbs, reps > 0 and at least 1 MiB");
    if (dev->recording) return fail(L0H_ERR_INVALID_OP, "the device is recording");
    bytes &= ~(size_t)15;
    void* buf = nullptr;
    unsigned* sink = nullptr;
    L0H_HIP_TRY(hipMalloc(&buf, bytes));
    hipError_t e = hipMalloc(&sink, 64);
    hipEvent_t a = nullptr, b = nullptr;
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    if (e == hipSuccess && zero_fill(dev->stream, buf, bytes)) e = hipErrorLaunchFailure;
    double best = 0.0;
    const size_t n16 = bytes / 16;
    // Launch shapes: 2, 4 and 8 blocks of 256 threads per CU; the best rate counts.
    for (int per_cu = 2; per_cu <= 8 && e == hipSuccess; per_cu *= 2) {
        const unsigned grid = (unsigned)(per_cu * std::max(1, dev->compute_units));
        read_stream_kernel<<<grid, 256, 0, dev->stream>>>(static_cast<const uint4*>(buf), n16, sink);  // warm-up
        e = hipEventRecord(a, dev->stream);
        for (int r = 0; r < reps && e == hipSuccess; r++) {
            read_stream_kernel<<<grid, 256, 0, dev->stream>>>(static_cast<const uint4*>(buf), n16, sink);
            e = hipGetLastError();
        }
        if (e == hipSuccess) e = hipEventRecord(b, dev->stream);
        if (e == hipSuccess) e = hipEventSynchronize(b);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
        if (e == hipSuccess && ms > 0.f) best = std::max(best, (double)bytes * reps / (ms * 1e-3) / 1e9);
    }
    (void)hipStreamSynchronize(dev->stream);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (sink) (void)hipFree(sink);
    (void)hipFree(buf);
    if (e != hipSuccess) return fail(L0H_ERR_DEVICE, std::string("read bandwidth probe: ") + hipGetErrorString(e));
    *gbs = best;
    return L0H_OK;
}

int l0h_synchronize(l0h_device* dev) {
    int st = use_device(dev);
    if (st) return st;
    if (dev->recording) return fail(L0H_ERR_INVALID_OP, "cannot synchronize while recording");
    L0H_HIP_TRY(hipStreamSynchronize(dev->stream));
    return L0H_OK;
}

}  // extern "C"
