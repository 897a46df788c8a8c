// kt_runtime.hip -- errors, device memory, streams, the per-stream workspace and
// the argument checks shared by every entry point of libkotensor_hip.so.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "kt_common.h"

namespace kt {

static thread_local char g_last_error[512] = "";

int32_t fail(int32_t status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int32_t hip_fail(hipError_t err, const char* what) {
    int32_t code = static_cast<int32_t>(err);
    if (code <= 0) code = 1;
    return fail(code, "%s failed: %s (%d)", what, hipGetErrorString(err), static_cast<int>(err));
}

namespace {
struct Block {
    void* ptr = nullptr;
    size_t bytes = 0;       // whole allocation
    size_t zbytes = 0;      // the zeroed accumulator region after the counters
    bool captured = false;  // handed to a kernel recorded into a graph
    int32_t fault = -1;     // the stream's slot of the fault words, once a kernel took it
};
std::mutex g_ws_mutex;
std::map<std::pair<int, hipStream_t>, Block> g_ws;
// Blocks replaced or orphaned while a recorded graph may still address them. A graph
// keeps the addresses it was recorded with, and graphs can outlive their stream, so
// these stay allocated until the process ends (each is smaller than its successor, so
// together they are bounded by a few times the largest workspace of the stream).
std::vector<void*> g_retired;
constexpr int MAX_DEVICES = 64;
int32_t g_cus[MAX_DEVICES] = {};  // compute units per device, 0 until asked

// A caller-provided workspace that replaces the per-stream one for the calls this
// thread makes while it is set (kt_qmatmul_noalloc), laid out like a stream's:
// counters, then zeroed fp64 accumulators, then the general area.
struct FixedWorkspace {
    char* ptr;
    size_t bytes;       // whole area
    size_t zero_bytes;  // the accumulator region after the counters
};
thread_local const FixedWorkspace* t_fixed = nullptr;
}  // namespace

// Each workspace starts with a COUNTER_BYTES region of uint32 counters and a region of
// fp64 accumulators, both zeroed when the allocation is made and left at zero by every
// kernel that uses them (the counter region's last words, from ROPE_CACHE_WORD, excepted:
// the decode attention's RoPE cache, whose entries a zeroed word marks as empty); the
// general area follows.
constexpr size_t COUNTER_BYTES = 64 << 10;
static_assert(ROPE_CACHE_WORD + 512 == COUNTER_BYTES / sizeof(uint32_t), "the RoPE cache ends the counter region");

static int32_t ensure(hipStream_t stream, size_t zbytes, size_t bytes, Block** out) {
    int device = 0;
    KT_HIP(hipGetDevice(&device));
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    KT_HIP(hipStreamIsCapturing(stream, &capture));
    const bool capturing = capture != hipStreamCaptureStatusNone;
    Block& b = g_ws[std::make_pair(device, stream)];
    const size_t zcap = zbytes > b.zbytes ? zbytes + zbytes / 4 : b.zbytes;
    if (zbytes > b.zbytes || b.bytes < COUNTER_BYTES + zcap + bytes) {
        // Growing needs an allocation and a zero fill, neither of which may be recorded:
        // a graph gets the workspace an eager call of the same shapes has sized.
        if (capturing)
            return fail(KT_ERR_STATE,
                        "the stream is capturing and its workspace is too small (needs %zu bytes, has %zu); "
                        "run one eager call of the same shapes on this stream before recording",
                        COUNTER_BYTES + zcap + bytes, b.bytes);
        const size_t need = COUNTER_BYTES + zcap + bytes;
        size_t want = need < (size_t(1) << 20) ? (size_t(1) << 20) : need + need / 4;
        if (b.ptr) {
            KT_HIP(hipStreamSynchronize(stream));
            if (b.captured) g_retired.push_back(b.ptr);  // a graph may still address it
            else KT_HIP(hipFree(b.ptr));
            const int32_t fault = b.fault;
            b = Block{};
            b.fault = fault;
        }
        KT_HIP(hipMalloc(&b.ptr, want));
        KT_HIP(hipMemsetAsync(b.ptr, 0, COUNTER_BYTES + zcap, stream));
        KT_HIP(hipStreamSynchronize(stream));
        b.bytes = want;
        b.zbytes = zcap;
    }
    if (capturing) b.captured = true;
    *out = &b;
    return KT_OK;
}

// The regions of the fixed workspace for a call that needs `doubles` accumulators and
// `bytes` of general area; a call that needs more is an argument error.
static int32_t fixed_regions(const FixedWorkspace& f, size_t doubles, size_t bytes, uint32_t** counters,
                             double** accs, void** general) {
    if (doubles * sizeof(double) > f.zero_bytes)
        return fail(KT_ERR_SHAPE, "the call needs %zu bytes of zeroed accumulators; the fixed workspace has %zu",
                    doubles * sizeof(double), f.zero_bytes);
    const size_t head = COUNTER_BYTES + f.zero_bytes;
    if (bytes > f.bytes - head)
        return fail(KT_ERR_SHAPE, "the call needs %zu bytes of workspace; the fixed workspace has %zu", bytes,
                    f.bytes - head);
    *counters = reinterpret_cast<uint32_t*>(f.ptr);
    *accs = reinterpret_cast<double*>(f.ptr + COUNTER_BYTES);
    *general = f.ptr + head;
    return KT_OK;
}

int32_t workspace(hipStream_t stream, size_t bytes, void** out) {
    if (t_fixed) {
        uint32_t* c;
        double* d;
        return fixed_regions(*t_fixed, 0, bytes, &c, &d, out);
    }
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Block* b = nullptr;
    int32_t status = ensure(stream, 0, bytes, &b);
    if (status) return status;
    *out = static_cast<char*>(b->ptr) + COUNTER_BYTES + b->zbytes;
    return KT_OK;
}

int32_t workspace_counters(hipStream_t stream, size_t bytes, size_t count, void** general, uint32_t** counters) {
    if (count > MAX_COUNTERS) return fail(KT_ERR_SHAPE, "too many reduction counters");
    if (t_fixed) {
        double* d;
        return fixed_regions(*t_fixed, 0, bytes, counters, &d, general);
    }
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Block* b = nullptr;
    int32_t status = ensure(stream, 0, bytes, &b);
    if (status) return status;
    *counters = static_cast<uint32_t*>(b->ptr);
    *general = static_cast<char*>(b->ptr) + COUNTER_BYTES + b->zbytes;
    return KT_OK;
}

int32_t workspace_accumulators(hipStream_t stream, size_t count, size_t doubles, uint32_t** counters, double** accs) {
    if (count > MAX_COUNTERS) return fail(KT_ERR_SHAPE, "too many reduction counters");
    if (t_fixed) {
        void* g;
        return fixed_regions(*t_fixed, doubles, 0, counters, accs, &g);
    }
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Block* b = nullptr;
    int32_t status = ensure(stream, doubles * sizeof(double), 0, &b);
    if (status) return status;
    *counters = static_cast<uint32_t*>(b->ptr);
    *accs = reinterpret_cast<double*>(static_cast<char*>(b->ptr) + COUNTER_BYTES);
    return KT_OK;
}

int32_t workspace_regions(hipStream_t stream, size_t doubles, size_t bytes, uint32_t** counters, double** accs,
                          void** general) {
    if (t_fixed) return fixed_regions(*t_fixed, doubles, bytes, counters, accs, general);
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Block* b = nullptr;
    int32_t status = ensure(stream, doubles * sizeof(double), bytes, &b);
    if (status) return status;
    *counters = static_cast<uint32_t*>(b->ptr);
    *accs = reinterpret_cast<double*>(static_cast<char*>(b->ptr) + COUNTER_BYTES);
    *general = static_cast<char*>(b->ptr) + COUNTER_BYTES + b->zbytes;
    return KT_OK;
}

int32_t cu_count() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return 256;
    if (device < 0 || device >= MAX_DEVICES) return 256;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if (g_cus[device] > 0) return g_cus[device];
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0)
        cus = 256;
    g_cus[device] = cus;
    return cus;
}

// ---- fault words of bounded waits ----------------------------------------------------
// One pinned host array mapped into every device; a stream takes the next slot the first
// time a waiting kernel is launched on it and keeps it (slots are not reused: a graph
// recorded on a stream keeps the address after the stream is gone; past FAULT_SLOTS
// streams, slots are shared, so a report may name a neighbouring stream too).
constexpr int32_t FAULT_SLOTS = 4096;
static int32_t* g_fault_host = nullptr;
static int32_t* g_fault_dev = nullptr;
static int32_t g_fault_next = 0;

static WaitLimits g_wait_limits{0u, 0};

WaitLimits wait_limits() { return g_wait_limits; }

int32_t stream_fault_word(hipStream_t stream, int32_t** dev_word) {
    *dev_word = nullptr;
    if (t_fixed) return KT_OK;  // the fixed workspace's calls run no waiting kernel
    int device = 0;
    KT_HIP(hipGetDevice(&device));
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if (!g_fault_host) {
        void* h = nullptr;
        KT_HIP(hipHostMalloc(&h, FAULT_SLOTS * sizeof(int32_t), hipHostMallocPortable | hipHostMallocMapped));
        memset(h, 0, FAULT_SLOTS * sizeof(int32_t));
        void* d = nullptr;
        const hipError_t err = hipHostGetDevicePointer(&d, h, 0);
        if (err != hipSuccess) {
            (void)hipHostFree(h);
            return hip_fail(err, "fault words: hipHostGetDevicePointer");
        }
        g_fault_host = static_cast<int32_t*>(h);
        g_fault_dev = static_cast<int32_t*>(d);
    }
    Block& b = g_ws[std::make_pair(device, stream)];
    if (b.fault < 0) b.fault = g_fault_next++ % FAULT_SLOTS;
    *dev_word = g_fault_dev + b.fault;
    return KT_OK;
}

// After a synchronization of `stream`: a give-up reported by a kernel on it is returned
// as KT_ERR_STATE, once, and the stream's counters and zeroed words are cleared, since
// a producer that arrived after its waiter gave up may have left flags or tagged words
// set that the next launch would take as its own.
static int32_t check_fault(hipStream_t stream) {
    int device = 0;
    KT_HIP(hipGetDevice(&device));
    int32_t code = 0;
    void* ptr = nullptr;
    size_t clear = 0;
    {
        std::lock_guard<std::mutex> lock(g_ws_mutex);
        auto it = g_ws.find(std::make_pair(device, stream));
        if (it == g_ws.end() || it->second.fault < 0 || !g_fault_host) return KT_OK;
        int32_t* word = g_fault_host + it->second.fault;
        code = __atomic_load_n(word, __ATOMIC_ACQUIRE);
        if (code == 0) return KT_OK;
        __atomic_store_n(word, 0, __ATOMIC_RELEASE);
        ptr = it->second.ptr;
        clear = COUNTER_BYTES + it->second.zbytes;
    }
    if (ptr) {
        KT_HIP(hipMemsetAsync(ptr, 0, clear, stream));
        KT_HIP(hipStreamSynchronize(stream));
    }
    return fail(KT_ERR_STATE,
                "a kernel's bounded wait gave up (code %d: %s); outputs of the calls on this stream since its last "
                "synchronization are not valid",
                code, code == FAULT_CHAIN_WAIT ? "a chained stage's input never arrived"
                      : code == FAULT_MERGE_WAIT ? "an attention split's sums never arrived"
                                                 : "unknown wait");
}

// ---- kt_qmatmul_noalloc's workspace -----------------------------------------------
// A file-scope device array, one copy per device (each GPU holds its own until the
// process ends). Host code never passes the array's name to a kernel: the name is a
// host-side stand-in, so each device's address is taken once with hipGetSymbolAddress
// and kept in g_scratch.
constexpr size_t SCRATCH_BYTES = 64 << 20;      // counters, accumulators and general area
constexpr size_t SCRATCH_ZERO_BYTES = 4 << 20;  // fp64 accumulators (half a million columns)
static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

struct ScratchSlot {
    char* ptr = nullptr;  // the device's address of `scratch`, once set up
};
ScratchSlot g_scratch[MAX_DEVICES];
std::mutex g_scratch_mutex;

__global__ void __launch_bounds__(256) clear_kernel(uint4* p, size_t n) {
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// The current device's scratch address. The first call on a device takes the address
// and clears the counters and accumulators (kernels leave them at zero after that); it
// runs the clear and waits for it, so it cannot be recorded into a graph.
static int32_t scratch_address(hipStream_t st, char** out) {
    int device = 0;
    KT_HIP(hipGetDevice(&device));
    if (device < 0 || device >= MAX_DEVICES) return fail(KT_ERR_ARGUMENT, "device %d out of range", device);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ScratchSlot& slot = g_scratch[device];
    if (!slot.ptr) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        KT_HIP(hipStreamIsCapturing(st, &capture));
        if (capture != hipStreamCaptureStatusNone)
            return fail(KT_ERR_STATE,
                        "kt_qmatmul_noalloc sets up its device array on its first call on a device, which cannot be "
                        "recorded; make one call outside a capture first");
        void* p = nullptr;
        KT_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        const size_t words = (COUNTER_BYTES + SCRATCH_ZERO_BYTES) / sizeof(uint4);
        clear_kernel<<<256, 256, 0, st>>>(static_cast<uint4*>(p), words);
        KT_LAUNCHED("kt_qmatmul_noalloc: clear");
        KT_HIP(hipStreamSynchronize(st));
        slot.ptr = static_cast<char*>(p);
    }
    *out = slot.ptr;
    return KT_OK;
}

int32_t view_weight(const kt_qweight* w, WeightView* v) {
    if (!w) return fail(KT_ERR_ARGUMENT, "weight is NULL");
    if (w->bits != 4 && w->bits != 8) return fail(KT_ERR_ARGUMENT, "bits must be 4 or 8, got %d", w->bits);
    if (w->group_size <= 0) return fail(KT_ERR_ARGUMENT, "groupSize must be positive");
    if (w->rows <= 0 || w->columns <= 0)
        return fail(KT_ERR_SHAPE, "QuantizedTensor needs a 2-D shape, got [%d, %d]", w->rows, w->columns);
    if (w->bits == 4 && !w->zeros) return fail(KT_ERR_ZEROS, "4-bit tensors need zero points");
    if (!w->qdata || !w->scales) return fail(KT_ERR_ARGUMENT, "weight has a NULL qdata or scales pointer");
    v->q = static_cast<const uint8_t*>(w->qdata);
    v->s = w->scales;
    v->z = reinterpret_cast<const int8_t*>(w->zeros);
    v->p = static_cast<const uint8_t*>(w->packed);
    v->K = w->rows;
    v->N = w->columns;
    v->bits = w->bits;
    v->g = w->group_size;
    v->G = (w->rows + w->group_size - 1) / w->group_size;
    v->bpr = w->bits == 4 ? (w->columns + w->columns % 2) / 2 : w->columns;
    int64_t qbytes = static_cast<int64_t>(v->K) * v->bpr;
    int64_t sbytes = static_cast<int64_t>(v->G) * v->N * 4;
    if (qbytes > INT32_MAX * 4LL || sbytes > INT32_MAX * 4LL)
        return fail(KT_ERR_SHAPE, "weight [%d, %d] is too large", v->K, v->N);
    return KT_OK;
}

}  // namespace kt

using namespace kt;

extern "C" {

int32_t kt_abi_version(void) { return KT_ABI_VERSION; }

int32_t kt_last_error(char* buf, size_t len) {
    if (!buf || len == 0) return KT_ERR_ARGUMENT;
    strncpy(buf, g_last_error, len - 1);
    buf[len - 1] = '\0';
    return KT_OK;
}

int32_t kt_device_count(int32_t* count) {
    if (!count) return fail(KT_ERR_ARGUMENT, "count is NULL");
    int n = 0;
    KT_HIP(hipGetDeviceCount(&n));
    *count = n;
    return KT_OK;
}

int32_t kt_set_device(int32_t device) {
    KT_HIP(hipSetDevice(device));
    return KT_OK;
}

// 0: automatic, 1: vector-ALU kernel, 2: MFMA row-block kernel, 3: MFMA wide-strip kernel,
// 4: column-strip latency kernel, 5: column-run kernel (packed copy).
static int32_t g_gemv_kind = 0;

int32_t kt_set_kernel_config(int32_t gemv_kind, int32_t gemv_vec, int32_t gemv_splits, int32_t gemv_waves,
                             int32_t gemv_reduce) {
    if (gemv_kind < 0 || gemv_kind > 5) return fail(KT_ERR_ARGUMENT, "gemv_kind must be 0 to 5, got %d", gemv_kind);
    if (gemv_vec != 0 && gemv_vec != 4 && gemv_vec != 8)
        return fail(KT_ERR_ARGUMENT, "gemv_vec must be 0, 4 or 8, got %d", gemv_vec);
    if (gemv_splits < 0) return fail(KT_ERR_ARGUMENT, "gemv_splits must be >= 0, got %d", gemv_splits);
    if (gemv_waves != 0 && gemv_waves != 2 && gemv_waves != 4 && gemv_waves != 8)
        return fail(KT_ERR_ARGUMENT, "gemv_waves must be 0, 2, 4 or 8, got %d", gemv_waves);
    if (gemv_reduce < 0 || gemv_reduce > 2)
        return fail(KT_ERR_ARGUMENT, "gemv_reduce must be 0, 1 or 2, got %d", gemv_reduce);
    set_gemv_config(gemv_vec, gemv_splits, gemv_waves == 2 ? 4 : gemv_waves);
    set_gemv_reduce_mode(gemv_reduce);
    set_gemv_mfma_config(gemv_splits, gemv_waves, gemv_reduce, gemv_kind == 1);
    set_gemv_wide_config(gemv_splits, gemv_waves);
    set_gemv_packed_config(gemv_splits, gemv_waves, gemv_vec);
    set_gemv_rows_packed_reduce(gemv_reduce);
    g_gemv_kind = gemv_kind;
    return KT_OK;
}

int32_t kt_dev_alloc(size_t bytes, void** ptr) {
    if (!ptr) return fail(KT_ERR_ARGUMENT, "ptr is NULL");
    *ptr = nullptr;
    if (bytes == 0) return KT_OK;
    KT_HIP(hipMalloc(ptr, bytes));
    return KT_OK;
}

int32_t kt_dev_free(void* ptr) {
    if (!ptr) return KT_OK;
    KT_HIP(hipFree(ptr));
    return KT_OK;
}

static int32_t copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, void* stream) {
    if (bytes == 0) return KT_OK;
    if (!dst || !src) return fail(KT_ERR_ARGUMENT, "copy with a NULL pointer");
    KT_HIP(hipMemcpyAsync(dst, src, bytes, kind, static_cast<hipStream_t>(stream)));
    if (kind == hipMemcpyDeviceToHost) KT_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return KT_OK;
}

int32_t kt_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    int32_t st = copy(dst, src, bytes, hipMemcpyHostToDevice, stream);
    if (st) return st;
    // The source is caller memory that may be reused once this returns.
    KT_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return KT_OK;
}

int32_t kt_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    const int32_t st = copy(dst, src, bytes, hipMemcpyDeviceToHost, stream);
    if (st) return st;
    if (bytes == 0) KT_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return check_fault(static_cast<hipStream_t>(stream));
}

int32_t kt_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    return copy(dst, src, bytes, hipMemcpyDeviceToDevice, stream);
}

int32_t kt_memset(void* dst, int32_t value, size_t bytes, void* stream) {
    if (bytes == 0) return KT_OK;
    if (!dst) return fail(KT_ERR_ARGUMENT, "memset of a NULL pointer");
    KT_HIP(hipMemsetAsync(dst, value, bytes, static_cast<hipStream_t>(stream)));
    return KT_OK;
}

int32_t kt_stream_create(void** stream) {
    if (!stream) return fail(KT_ERR_ARGUMENT, "stream is NULL");
    hipStream_t s = nullptr;
    KT_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return KT_OK;
}

int32_t kt_stream_destroy(void* stream) {
    if (!stream) return KT_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    KT_HIP(hipStreamSynchronize(s));
    {
        int device = 0;
        KT_HIP(hipGetDevice(&device));
        std::lock_guard<std::mutex> lock(g_ws_mutex);
        auto it = g_ws.find(std::make_pair(device, s));
        if (it != g_ws.end()) {
            // A graph recorded on this stream may be replayed on another one later.
            if (it->second.ptr && it->second.captured) g_retired.push_back(it->second.ptr);
            else if (it->second.ptr) KT_HIP(hipFree(it->second.ptr));
            g_ws.erase(it);
        }
    }
    KT_HIP(hipStreamDestroy(s));
    return KT_OK;
}

int32_t kt_stream_sync(void* stream) {
    KT_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return check_fault(static_cast<hipStream_t>(stream));
}

int32_t kt_debug_wait_limits(uint32_t spin_limit, int32_t withhold) {
    if (withhold != 0 && withhold != 1) return fail(KT_ERR_ARGUMENT, "withhold must be 0 or 1, got %d", withhold);
    g_wait_limits = WaitLimits{spin_limit, withhold};
    return KT_OK;
}

int32_t kt_graph_begin(void* stream) {
    if (!stream) return fail(KT_ERR_ARGUMENT, "the null stream cannot be captured; create a stream");
    KT_HIP(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal));
    return KT_OK;
}

int32_t kt_graph_end(void* stream, void** graph) {
    if (!stream || !graph) return fail(KT_ERR_ARGUMENT, "stream or graph is NULL");
    *graph = nullptr;
    hipGraph_t g = nullptr;
    KT_HIP(hipStreamEndCapture(static_cast<hipStream_t>(stream), &g));
    hipGraphExec_t exec = nullptr;
    const hipError_t err = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (err != hipSuccess) return hip_fail(err, "hipGraphInstantiate");
    *graph = exec;
    return KT_OK;
}

int32_t kt_graph_launch(void* graph, void* stream) {
    if (!graph) return fail(KT_ERR_ARGUMENT, "graph is NULL");
    KT_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), static_cast<hipStream_t>(stream)));
    return KT_OK;
}

int32_t kt_graph_destroy(void* graph) {
    if (graph) KT_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)));
    return KT_OK;
}

int32_t kt_qweight_layout(int32_t rows, int32_t columns, int32_t bits, int32_t group_size,
                          int32_t has_zeros, int64_t* out4) {
    if (!out4) return fail(KT_ERR_ARGUMENT, "out is NULL");
    if (bits != 4 && bits != 8) return fail(KT_ERR_ARGUMENT, "bits must be 4 or 8, got %d", bits);
    if (group_size <= 0) return fail(KT_ERR_ARGUMENT, "groupSize must be positive");
    if (rows <= 0 || columns <= 0) return fail(KT_ERR_SHAPE, "QuantizedTensor needs a 2-D shape, got [%d, %d]", rows, columns);
    int64_t groups = (rows + static_cast<int64_t>(group_size) - 1) / group_size;
    int64_t stored = bits == 4 ? columns + columns % 2 : columns;
    int64_t bpr = bits == 4 ? stored / 2 : stored;
    out4[0] = groups;
    out4[1] = stored;
    out4[2] = bpr;
    out4[3] = rows * bpr + groups * columns * 4 + (has_zeros ? groups * columns : 0);
    return KT_OK;
}

int32_t kt_qweight_check(const kt_qweight* w) {
    WeightView v;
    return view_weight(w, &v);
}

int32_t kt_qweight_packed_bytes(int32_t rows, int32_t columns, int32_t bits, int32_t group_size, int64_t* bytes) {
    if (!bytes) return fail(KT_ERR_ARGUMENT, "bytes is NULL");
    if (bits != 4 && bits != 8) return fail(KT_ERR_ARGUMENT, "bits must be 4 or 8, got %d", bits);
    if (group_size <= 0) return fail(KT_ERR_ARGUMENT, "groupSize must be positive");
    if (rows <= 0 || columns <= 0) return fail(KT_ERR_SHAPE, "QuantizedTensor needs a 2-D shape, got [%d, %d]", rows, columns);
    *bytes = packed_bytes(rows, columns, bits, group_size);
    return KT_OK;
}

int32_t kt_qweight_pack(const kt_qweight* w, void* packed, void* stream) {
    WeightView v;
    int32_t status = view_weight(w, &v);
    if (status) return status;
    if (!packed) return fail(KT_ERR_ARGUMENT, "packed is NULL");
    if (!aligned(packed, 16)) return fail(KT_ERR_ARGUMENT, "packed must be 16-byte aligned");
    return launch_pack(v, packed, static_cast<hipStream_t>(stream));
}

constexpr uint32_t NAN_SLOTS = 1024;  // quantize calls that may be in flight at once

int32_t kt_quantize(const float* data, int32_t rows, int32_t columns, int32_t bits, int32_t group_size,
                    void* qdata, float* scales, uint8_t* zeros, void* stream) {
    if (bits != 4 && bits != 8) return fail(KT_ERR_ARGUMENT, "bits must be 4 or 8, got %d", bits);
    if (group_size <= 0) return fail(KT_ERR_ARGUMENT, "groupSize must be positive");
    if (rows <= 0 || columns <= 0) return fail(KT_ERR_SHAPE, "QuantizedTensor needs a 2-D shape, got [%d, %d]", rows, columns);
    if (!data || !qdata || !scales) return fail(KT_ERR_ARGUMENT, "quantize with a NULL pointer");
    if (bits == 4 && !zeros) return fail(KT_ERR_ZEROS, "4-bit tensors need zero points");
    if (bits == 8 && zeros) return fail(KT_ERR_ARGUMENT, "8-bit quantize writes no zero points; pass NULL");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // The NaN report (the reference throws from inside quantize): a pinned host array of
    // NAN_SLOTS flags, one per call in flight, never cleared. Each call takes the next
    // epoch (nonzero) and its slot; the kernel stores the epoch there when it meets a NaN,
    // and the call reads the slot once the stream has synchronized. No clearing launch and
    // no copy: the call costs the kernel and the synchronization.
    static std::once_flag once;
    static int32_t* host_slots = nullptr;
    static int32_t* dev_slots = nullptr;
    static hipError_t init_err = hipSuccess;
    std::call_once(once, [] {
        void* h = nullptr;
        init_err = hipHostMalloc(&h, NAN_SLOTS * sizeof(int32_t), hipHostMallocPortable | hipHostMallocMapped);
        if (init_err != hipSuccess) return;
        memset(h, 0, NAN_SLOTS * sizeof(int32_t));
        void* d = nullptr;
        init_err = hipHostGetDevicePointer(&d, h, 0);
        if (init_err != hipSuccess) return;
        host_slots = static_cast<int32_t*>(h);
        dev_slots = static_cast<int32_t*>(d);
    });
    if (init_err != hipSuccess) return hip_fail(init_err, "quantize: pinned NaN flags");
    static std::atomic<uint32_t> epochs{0};
    uint32_t e = 0;
    while (e == 0) e = (epochs.fetch_add(1) + 1) & 0x7FFFFFFFu;
    const int32_t epoch = static_cast<int32_t>(e);
    int32_t* slot = dev_slots + (e % NAN_SLOTS);
    int32_t status = launch_quantize(data, rows, columns, bits, group_size, static_cast<uint8_t*>(qdata), scales,
                                     reinterpret_cast<int8_t*>(zeros), slot, epoch, st);
    if (status) return status;
    KT_HIP(hipStreamSynchronize(st));
    if (__atomic_load_n(host_slots + (e % NAN_SLOTS), __ATOMIC_ACQUIRE) == epoch)
        return fail(KT_ERR_NAN, "Cannot round NaN value.");
    return KT_OK;
}

static int32_t qmatmul_impl(const float* a, int32_t m, const kt_qweight* w, float* c, int32_t accumulate,
                            float alpha, const float* bias, void* stream) {
    WeightView v;
    int32_t status = view_weight(w, &v);
    if (status) return status;
    if (m < 0) return fail(KT_ERR_ARGUMENT, "Negative row count %d", m);
    if (m == 0) return KT_OK;
    if (!a || !c) return fail(KT_ERR_ARGUMENT, "matmul with a NULL input or output");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const float* biases[1] = {bias};
    if ((g_gemv_kind == 0 || g_gemv_kind == 5) && gemv_packed_supported(a, m, v, c))
        return launch_gemv_packed(a, &v, &c, biases, 1, accumulate, alpha, st);
    if (g_gemv_kind == 0 && m >= 2 && gemv_packed_supported(a, 1, v, c) && gemv_packed_rows_rep_preferred(m, &v, 1))
        return launch_gemv_packed_rows_rep(a, m, v, c, bias, accumulate, alpha, st);
    if ((g_gemv_kind == 5 || (g_gemv_kind == 0 && gemv_rows_packed_preferred(v))) &&
        gemv_rows_packed_supported(a, m, v, c))
        return launch_gemv_rows_packed(a, m, &v, &c, biases, 1, accumulate, alpha, st);
    if ((g_gemv_kind == 4 || (g_gemv_kind == 0 && gemv_strip_preferred(&v, 1))) && gemv_strip_supported(a, m, v, c))
        return launch_gemv_strip(a, &v, &c, biases, 1, accumulate, alpha, st);
    if ((g_gemv_kind == 3 || (g_gemv_kind == 0 && gemv_wide_preferred(&v, 1))) && gemv_wide_supported(a, m, v, c))
        return launch_gemv_wide(a, &v, &c, biases, 1, accumulate, alpha, st);
    if (m <= 16 && gemv_mfma_supported(a, m, v, c)) return launch_gemv_mfma(a, m, &v, &c, biases, 1, accumulate, alpha, st);
    if (m == 1 && gemv_supported(a, v, c)) return launch_gemv(a, v, c, accumulate, alpha, bias, st);
    if (m > 1 && gemm_supported(a, m, v, c) && (!bias || aligned(bias, 16)))
        return launch_gemm(a, m, v, c, accumulate, alpha, bias, st);
    return launch_generic(a, m, v, c, accumulate, alpha, bias, st);
}

int32_t kt_qmatmul_group(const float* a, int32_t m, const kt_qweight* weights, int32_t count, float* const* outputs,
                         const float* const* biases, int32_t accumulate, float alpha, void* stream) {
    if (count < 0) return fail(KT_ERR_ARGUMENT, "Negative weight count %d", count);
    if (count == 0) return KT_OK;
    if (!weights || !outputs) return fail(KT_ERR_ARGUMENT, "group with a NULL weight or output array");
    if (m < 0) return fail(KT_ERR_ARGUMENT, "Negative row count %d", m);
    WeightView views[4];
    for (int32_t start = 0; start < count; start += 4) {
        const int32_t n = count - start < 4 ? count - start : 4;
        bool fast = m == 1 && a != nullptr;
        bool mfma = m >= 1 && m <= 16 && a != nullptr;
        bool wide = (g_gemv_kind == 0 || g_gemv_kind == 3) && a != nullptr;
        bool strip = (g_gemv_kind == 0 || g_gemv_kind == 4) && a != nullptr;
        bool packed = (g_gemv_kind == 0 || g_gemv_kind == 5) && a != nullptr;
        bool rows_packed = packed && m >= 2;
        bool rep = g_gemv_kind == 0 && m >= 2 && a != nullptr;  // rows as one-row products
        bool gemm = m > 2 && a != nullptr;
        for (int32_t i = 0; i < n; ++i) {
            int32_t status = view_weight(&weights[start + i], &views[i]);
            if (status) return status;
            const WeightView& v = views[i];
            if (v.K != views[0].K || v.bits != views[0].bits || v.g != views[0].g)
                return fail(KT_ERR_SHAPE, "grouped weights must share rows, bits and group size");
            if (!outputs[start + i]) return fail(KT_ERR_ARGUMENT, "group output %d is NULL", start + i);
            const float* b = biases ? biases[start + i] : nullptr;
            fast = fast && gemv_supported(a, v, outputs[start + i]) && (!b || aligned(b, 16));
            mfma = mfma && gemv_mfma_supported(a, m, v, outputs[start + i]);
            wide = wide && gemv_wide_supported(a, m, v, outputs[start + i]);
            strip = strip && gemv_strip_supported(a, m, v, outputs[start + i]) && (!b || aligned(b, 4));
            packed = packed && gemv_packed_supported(a, m, v, outputs[start + i]);
            rep = rep && gemv_packed_supported(a, 1, v, outputs[start + i]) &&
                  (v.z != nullptr) == (views[0].z != nullptr);
            rows_packed = rows_packed && gemv_rows_packed_supported(a, m, v, outputs[start + i]) &&
                          (g_gemv_kind == 5 || gemv_rows_packed_preferred(v));
            gemm = gemm && gemm_supported(a, m, v, outputs[start + i]) && (!b || aligned(b, 16)) &&
                   (v.z != nullptr) == (views[0].z != nullptr);
        }
        if (m == 0) continue;
        if (!a) return fail(KT_ERR_ARGUMENT, "matmul with a NULL input");
        hipStream_t st = static_cast<hipStream_t>(stream);
        int32_t status = KT_OK;
        if (strip && g_gemv_kind == 0 && !gemv_strip_preferred(views, n)) strip = false;
        if (wide && g_gemv_kind == 0 && !gemv_wide_preferred(views, n)) wide = false;
        if (rep && !gemv_packed_rows_rep_preferred(m, views, n)) rep = false;
        if (packed) {
            status = launch_gemv_packed(a, views, outputs + start, biases ? biases + start : nullptr, n, accumulate,
                                        alpha, st);
        } else if (rep) {
            status = launch_gemv_packed_group_rep(a, m, views, outputs + start, biases ? biases + start : nullptr, n,
                                                  accumulate, alpha, st);
        } else if (rows_packed) {
            status = launch_gemv_rows_packed(a, m, views, outputs + start, biases ? biases + start : nullptr, n,
                                             accumulate, alpha, st);
        } else if (strip) {
            status = launch_gemv_strip(a, views, outputs + start, biases ? biases + start : nullptr, n, accumulate, alpha, st);
        } else if (wide) {
            status = launch_gemv_wide(a, views, outputs + start, biases ? biases + start : nullptr, n, accumulate, alpha, st);
        } else if (mfma) {
            status = launch_gemv_mfma(a, m, views, outputs + start, biases ? biases + start : nullptr, n, accumulate,
                                      alpha, st);
        } else if (fast) {
            status = launch_gemv_group(a, views, outputs + start, biases ? biases + start : nullptr, n, accumulate, alpha, st);
        } else if (gemm) {
            status = launch_gemm_group(a, m, views, outputs + start, biases ? biases + start : nullptr, n, accumulate,
                                       alpha, st);
        } else {
            for (int32_t i = 0; i < n && status == KT_OK; ++i)
                status = qmatmul(a, m, &weights[start + i], outputs[start + i], accumulate, alpha,
                                 biases ? biases[start + i] : nullptr, stream);
        }
        if (status) return status;
    }
    return KT_OK;
}

int32_t kt_qmatmul(const float* a, int32_t m, const kt_qweight* w, float* c, int32_t accumulate, float alpha,
                   void* stream) {
    return qmatmul_impl(a, m, w, c, accumulate, alpha, nullptr, stream);
}

int32_t kt_qmatmul_noalloc(const float* a, int32_t m, const kt_qweight* w, float* c, int32_t accumulate, float alpha,
                           void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    char* base = nullptr;
    if (int32_t status = scratch_address(st, &base)) return status;
    const FixedWorkspace fixed{base, SCRATCH_BYTES, SCRATCH_ZERO_BYTES};
    struct Scope {
        explicit Scope(const FixedWorkspace* f) { t_fixed = f; }
        ~Scope() { t_fixed = nullptr; }
    } scope(&fixed);
    return qmatmul_impl(a, m, w, c, accumulate, alpha, nullptr, stream);
}

int32_t kt_qlinear_forward(const float* a, int32_t m, const kt_qweight* w, const float* bias, float* out,
                           void* stream) {
    return qmatmul_impl(a, m, w, out, 0, 1.0f, bias, stream);
}

int32_t kt_qmatmul_transposed(const float* dy, int32_t m, const kt_qweight* w, float* dx, int32_t accumulate,
                              void* stream) {
    WeightView v;
    int32_t status = view_weight(w, &v);
    if (status) return status;
    if (m < 0) return fail(KT_ERR_ARGUMENT, "Negative row count %d", m);
    if (m == 0) return KT_OK;
    if (!dy || !dx) return fail(KT_ERR_ARGUMENT, "matmul with a NULL input or output");
    return launch_transposed(dy, m, v, dx, accumulate, static_cast<hipStream_t>(stream));
}

int32_t kt_dequantize_rows(const kt_qweight* w, const int32_t* rows, int32_t count, float* out, void* stream) {
    WeightView v;
    int32_t status = view_weight(w, &v);
    if (status) return status;
    if (count < 0) return fail(KT_ERR_ARGUMENT, "Negative count %d", count);
    if (count == 0) return KT_OK;
    if (!rows || !out) return fail(KT_ERR_ARGUMENT, "dequantize with a NULL pointer");
    return launch_dequantize_rows(v, rows, count, out, static_cast<hipStream_t>(stream));
}

int32_t kt_dequantize_columns(const kt_qweight* w, const int32_t* columns, int32_t count, float* out,
                              void* stream) {
    WeightView v;
    int32_t status = view_weight(w, &v);
    if (status) return status;
    if (count < 0) return fail(KT_ERR_ARGUMENT, "Negative count %d", count);
    if (count == 0) return KT_OK;
    if (!columns || !out) return fail(KT_ERR_ARGUMENT, "dequantize with a NULL pointer");
    return launch_dequantize_columns(v, columns, count, out, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace kt {

int32_t gemv_kind() { return g_gemv_kind; }

int32_t qmatmul(const float* a, int32_t m, const kt_qweight* w, float* c, int32_t accumulate, float alpha,
                const float* bias, void* stream) {
    return qmatmul_impl(a, m, w, c, accumulate, alpha, bias, stream);
}

}  // namespace kt
