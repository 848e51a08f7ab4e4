// mt_shim.cpp -- native C-ABI shim for the MI355X backend (declarations and
// contract: include/metellus_hip.h).
//
// Replaces the reference's Metal backend (reference: src/metal_backend.mm):
//   * a buffer registry of stream-ordered device allocations (hipMallocAsync /
//     hipFreeAsync), opaque u64 handles starting at 1;
//   * hiprtc compilation of generated kernels with an in-memory and on-disk
//     code-object cache keyed by the exact (source, function, options, target)
//     text -- the reference recompiled MSL on every dispatch
//     (metal_backend.mm:188-207);
//   * hipModuleLaunchKernel on a single stream, asynchronous unless timed --
//     the reference waited after every dispatch (metal_backend.mm:226-227);
//   * mt_launch_noalloc: the same launch for callers that cannot allocate,
//     with stream-K kernels' workspace in a static device array (`scratch`).
//
// Its only device code is that array and a word-clearing kernel; every
// compute kernel is generated and compiled at run time.

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <sys/stat.h>
#include <unistd.h>
#include <unordered_map>
#include <vector>

#include "../../include/metellus_hip.h"

namespace {

thread_local std::string g_error;

int fail(const std::string& msg) {
    g_error = msg;
    return 1;
}

#define MT_HIP(call)                                                                      \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess) {                                                           \
            return fail(std::string(#call) + " failed: " + hipGetErrorString(e_));        \
        }                                                                                 \
    } while (0)

constexpr int kMaxDims = 16;
struct DimsArg {
    uint32_t v[kMaxDims];
};

struct Buffer {
    void* ptr;
    size_t nbytes;
    size_t cap;  // bytes of the block behind ptr (>= nbytes; the device cache's size class)
};

struct Kernel {
    hipModule_t module;
    hipFunction_t function;
};

constexpr int kStages = 3;  // page-locked staging buffers of a pageable transfer

struct State {
    std::mutex mu;
    bool ready = false;
    hipStream_t stream = nullptr;
    hipEvent_t ev_start = nullptr;
    hipEvent_t ev_stop = nullptr;
    hipEvent_t marks[16] = {};  // mt_mark / mt_mark_elapsed
    std::string arch;  // full target id of device 0
    int cu_count = 0;
    int clock_khz = 0;
    std::unordered_map<uint64_t, Buffer> buffers;
    uint64_t next_buffer = 1;
    std::vector<Kernel> kernels;                       // handle = index + 1
    std::unordered_map<std::string, uint64_t> by_key;  // exact key -> handle
    uint64_t compiled = 0;
    uint64_t hits = 0;
    // Pinned host blocks: capacity of every live or cached block, and the
    // cached (returned) ones by capacity.
    std::unordered_map<void*, size_t> host_cap;
    std::multimap<size_t, void*> host_free;
    size_t host_cached = 0;
    // Freed device blocks kept for reuse, by capacity (see mt_free).
    std::multimap<size_t, void*> dev_free;
    size_t dev_cached = 0;
    size_t dev_cache_limit = 0;
    // Allocations the shim asked the runtime for: device blocks
    // (hipMallocAsync) and page-locked host blocks (hipHostMalloc).
    uint64_t device_allocs = 0;
    uint64_t host_allocs = 0;
    // Workspace of stream-K kernels (a registry buffer the shim owns).
    uint64_t ws_handle = 0;
    size_t ws_bytes = 0;
    // Staging ring for transfers between pageable host memory and the device.
    void* stage[kStages] = {};
    hipEvent_t stage_ev[kStages] = {};
    // Device address of `scratch` per device id, from hipGetSymbolAddress
    // with that device current (the shim runs on device 0: entry 0).
    void* scratch_ptr[16] = {};
};

// Workspace layout shared with the device library (MT_WS_HEAD): flag words,
// the last of them the error word, then the partial tiles.
constexpr size_t kWsHeadBytes = 1024 * sizeof(uint32_t);
constexpr size_t kWsErrorOffset = 1023 * sizeof(uint32_t);

// ---- static scratch of the allocation-free launch ---------------------------
//
// The workspace of stream-K kernels launched by mt_launch_noalloc: the
// 4 KiB flag head, then partial tiles -- 64 MiB holds one 256x256 fp32 tile
// (or two 256x128 accumulator sets) for each of 256 persistent workgroups,
// what the C4 matmuls use.  Each device the library runs on holds its own
// copy from module load until the process ends.  In host code `scratch` is
// only a symbol: its device address comes from hipGetSymbolAddress (at
// init) and is the only form passed to kernels.
constexpr size_t kScratchBytes = kWsHeadBytes + (size_t(64) << 20);
static __device__ __align__(256) uint32_t scratch[kScratchBytes / sizeof(uint32_t)];

// Zero n words (vector stores, one per lane): the scratch head before each
// allocation-free stream-K launch.  A kernel instead of hipMemsetAsync, so
// the launch stays correct when a caller captures it in a graph.
__global__ void mt_clear_words(uint32_t* p, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

constexpr int kMaxLaunchBuffers = 64;

constexpr size_t kHostGranule = size_t(64) << 10;     // pinned blocks are multiples of 64 KiB
constexpr size_t kHostCacheLimit = size_t(1) << 30;   // at most 1 GiB of returned blocks kept

// Device block cache.  Returning device memory to the driver makes every
// host<->device copy of the next ~50 ms run at half speed on MI355X (a
// 256 MiB download: 4.7 ms -> 8.7-10 ms after a free of 256-768 MiB,
// measured with C3 run()s back to back; the copies themselves are unchanged).
// hipFreeAsync returns the memory at once although the default pool's release
// threshold is set to keep it (its reserved size drops to 0), so freed blocks
// stay here instead and serve later allocations of their size class.  Reuse
// is stream-ordered like hipFreeAsync: every copy, fill and launch of the shim
// runs on its one stream, so work queued before a free finishes before the
// block's next owner touches it.
constexpr size_t kDevGranule = size_t(2) << 20;       // blocks >= 2 MiB: multiples of 2 MiB
constexpr size_t kDevSmallGranule = 256;               // smaller blocks: multiples of 256 B
// At most 8 GiB (or a sixteenth of the device) of freed blocks are kept by
// default: several times the working set of the largest program here (C4,
// ~1.3 GB), little enough that another allocator in the process or another
// process on the GPU is not starved.  MT_DEVICE_CACHE_MB overrides it (0:
// every free goes back to the driver); mt_trim empties the cache.
constexpr size_t kDevCacheMax = size_t(8) << 30;

size_t dev_cache_limit(size_t total_mem) {
    if (const char* env = std::getenv("MT_DEVICE_CACHE_MB")) {
        char* end = nullptr;
        const unsigned long long mb = std::strtoull(env, &end, 10);
        if (end != env && *end == '\0') return static_cast<size_t>(mb) << 20;
    }
    return std::min(kDevCacheMax, total_mem / 16);
}

size_t dev_capacity(size_t nbytes) {
    const size_t g = nbytes >= kDevGranule ? kDevGranule : kDevSmallGranule;
    return (nbytes + g - 1) / g * g;
}

State& state() {
    static State s;
    return s;
}

// ---- staged host transfers ----------------------------------------------------
//
// A copy between pageable host memory and the device runs at ~30 GB/s
// host-to-device and ~17 GB/s device-to-host on MI355X (the driver stages it
// through its own pinned buffer, one thread); page-locked memory moves at
// ~57 GB/s each way.  Large transfers from or to pageable memory are therefore
// cut into chunks that go through a ring of page-locked staging buffers: a
// few host threads copy chunk i into (or out of) its staging buffer while the
// DMA engine moves chunk i-1 (measured: 4 threads copy 83 GB/s on the box).
// Page-locked host pointers (mt_host_alloc blocks) keep the direct copy.

constexpr size_t kStageChunk = size_t(16) << 20;
constexpr size_t kStageMin = size_t(4) << 20;  // smaller transfers copy directly
constexpr int kCopyThreads = 3;                // plus the calling thread

// Persistent workers for parallel memcpy; one caller at a time (the shim's
// state mutex is held around every transfer).
class CopyPool {
  public:
    CopyPool() {
        for (int i = 0; i < kCopyThreads; ++i) workers_.emplace_back([this] { loop(); });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : workers_) t.join();
    }
    // memcpy(dst, src, n), split over the workers and the calling thread.
    void copy(void* dst, const void* src, size_t n) {
        const size_t parts = workers_.size() + 1;
        size_t per = (n + parts - 1) / parts;
        per = (per + 4095) & ~size_t(4095);
        char* d = static_cast<char*>(dst);
        const char* sp = static_cast<const char*>(src);
        size_t first = std::min(per, n);
        {
            std::lock_guard<std::mutex> lk(mu_);
            for (size_t off = first; off < n; off += per) {
                jobs_.push_back(Job{d + off, sp + off, std::min(per, n - off)});
                ++pending_;
            }
        }
        cv_.notify_all();
        std::memcpy(d, sp, first);
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [this] { return pending_ == 0; });
    }

  private:
    struct Job {
        char* dst;
        const char* src;
        size_t n;
    };
    void loop() {
        for (;;) {
            Job j;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [this] { return stop_ || !jobs_.empty(); });
                if (jobs_.empty()) return;  // stop_ and nothing left
                j = jobs_.front();
                jobs_.pop_front();
            }
            std::memcpy(j.dst, j.src, j.n);
            std::lock_guard<std::mutex> lk(mu_);
            if (--pending_ == 0) done_.notify_all();
        }
    }
    std::vector<std::thread> workers_;
    std::deque<Job> jobs_;
    std::mutex mu_;
    std::condition_variable cv_, done_;
    size_t pending_ = 0;
    bool stop_ = false;
};

CopyPool& copy_pool() {
    static CopyPool pool;
    return pool;
}

bool is_pinned(const void* p) {
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();  // pageable memory is reported as an error; clear it
        return false;
    }
    return attr.type == hipMemoryTypeHost;
}

// Caller holds s.mu and has initialised the device.  All or nothing: the
// ring is installed only when every buffer and event was created.
int ensure_staging(State& s) {
    if (s.stage[0]) return 0;
    void* buf[kStages] = {};
    hipEvent_t ev[kStages] = {};
    hipError_t e = hipSuccess;
    for (int b = 0; b < kStages && e == hipSuccess; ++b) {
        e = hipHostMalloc(&buf[b], kStageChunk, hipHostMallocDefault);
        if (e == hipSuccess) ++s.host_allocs;
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev[b], hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        for (int b = 0; b < kStages; ++b) {
            if (buf[b]) (void)hipHostFree(buf[b]);
            if (ev[b]) (void)hipEventDestroy(ev[b]);
        }
        return fail(std::string("staging buffers for a pageable transfer: ") + hipGetErrorString(e));
    }
    for (int b = 0; b < kStages; ++b) s.stage[b] = buf[b], s.stage_ev[b] = ev[b];
    return 0;
}

int staged_upload(State& s, char* dst, const char* src, size_t n) {
    if (ensure_staging(s)) return 1;
    for (size_t i = 0, off = 0; off < n; ++i, off += kStageChunk) {
        const int b = static_cast<int>(i % kStages);
        const size_t len = std::min(kStageChunk, n - off);
        if (i >= static_cast<size_t>(kStages)) MT_HIP(hipEventSynchronize(s.stage_ev[b]));  // its last DMA is done
        copy_pool().copy(s.stage[b], src + off, len);
        MT_HIP(hipMemcpyAsync(dst + off, s.stage[b], len, hipMemcpyHostToDevice, s.stream));
        MT_HIP(hipEventRecord(s.stage_ev[b], s.stream));
    }
    MT_HIP(hipStreamSynchronize(s.stream));
    return 0;
}

int staged_download(State& s, char* dst, const char* src, size_t n) {
    if (ensure_staging(s)) return 1;
    const size_t chunks = (n + kStageChunk - 1) / kStageChunk;
    auto issue = [&](size_t i) -> int {
        const int b = static_cast<int>(i % kStages);
        const size_t off = i * kStageChunk;
        MT_HIP(hipMemcpyAsync(s.stage[b], src + off, std::min(kStageChunk, n - off), hipMemcpyDeviceToHost, s.stream));
        MT_HIP(hipEventRecord(s.stage_ev[b], s.stream));
        return 0;
    };
    for (size_t i = 0; i < std::min(chunks, static_cast<size_t>(kStages)); ++i)
        if (issue(i)) return 1;
    for (size_t i = 0; i < chunks; ++i) {
        const int b = static_cast<int>(i % kStages);
        const size_t off = i * kStageChunk;
        MT_HIP(hipEventSynchronize(s.stage_ev[b]));
        copy_pool().copy(dst + off, s.stage[b], std::min(kStageChunk, n - off));
        if (i + kStages < chunks && issue(i + kStages)) return 1;  // reuses buffer b, now copied out
    }
    return 0;
}

// Caller holds s.mu.
int init_locked(State& s) {
    if (s.ready) return 0;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        return fail(std::string("no HIP device available: ") +
                    (e != hipSuccess ? hipGetErrorString(e) : "device count is 0"));
    }
    MT_HIP(hipSetDevice(0));
    MT_HIP(hipGetSymbolAddress(&s.scratch_ptr[0], HIP_SYMBOL(scratch)));
    hipDeviceProp_t prop;
    MT_HIP(hipGetDeviceProperties(&prop, 0));
    s.arch = prop.gcnArchName;
    s.cu_count = prop.multiProcessorCount;
    s.clock_khz = prop.clockRate;
    s.dev_cache_limit = dev_cache_limit(static_cast<size_t>(prop.totalGlobalMem));
    MT_HIP(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
    // Timing-only events: without the system-scope release at record time
    // (an L2 write-back of the kernel's dirty lines), the bracket measures
    // the kernel and not the fence -- measured on MI355X, a 53 us stream
    // kernel reads 56.4 us with default events, 54.1 us with these.  Host
    // visibility does not depend on them: mt_read copies on the stream and
    // synchronises it.
    MT_HIP(hipEventCreateWithFlags(&s.ev_start, hipEventDisableSystemFence));
    MT_HIP(hipEventCreateWithFlags(&s.ev_stop, hipEventDisableSystemFence));
    for (auto& m : s.marks) MT_HIP(hipEventCreateWithFlags(&m, hipEventDisableSystemFence));
    // Keep memory released by hipFreeAsync in the device's pool instead of
    // returning it at each synchronisation, so buffers of repeated runs are
    // served from the pool.
    hipMemPool_t pool = nullptr;
    if (hipDeviceGetDefaultMemPool(&pool, 0) == hipSuccess && pool != nullptr) {
        uint64_t keep = ~uint64_t(0);
        MT_HIP(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep));
    }
    s.ready = true;
    return 0;
}

// ---- hiprtc -----------------------------------------------------------------

std::vector<std::string> split_options(const char* opts) {
    std::vector<std::string> out;
    if (opts == nullptr) return out;
    std::string cur;
    for (const char* p = opts; *p; ++p) {
        if (*p == ' ' || *p == '\t' || *p == '\n') {
            if (!cur.empty()) out.push_back(cur), cur.clear();
        } else {
            cur.push_back(*p);
        }
    }
    if (!cur.empty()) out.push_back(cur);
    return out;
}

std::vector<std::string> full_options(const std::string& target, const char* extra) {
    std::vector<std::string> o = {
        "--offload-arch=" + target,
        "-O3",
        "-std=c++17",
        "-ffp-contract=off",
        // Packed fp32 VALU forms are disabled for every kernel on this pool.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    };
    for (auto& x : split_options(extra)) o.push_back(x);
    return o;
}

int rtc_compile(const std::string& source, const std::vector<std::string>& options,
                std::vector<char>* code) {
    hiprtcProgram prog;
    hiprtcResult r = hiprtcCreateProgram(&prog, source.c_str(), "metellus_kernel.hip", 0, nullptr, nullptr);
    if (r != HIPRTC_SUCCESS) return fail(std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
    std::vector<const char*> argv;
    for (auto& s : options) argv.push_back(s.c_str());
    r = hiprtcCompileProgram(prog, static_cast<int>(argv.size()), argv.data());
    if (r != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string log(n, '\0');
        if (n) hiprtcGetProgramLog(prog, &log[0]);
        hiprtcDestroyProgram(&prog);
        return fail(std::string("hiprtc compile failed: ") + hiprtcGetErrorString(r) + "\n" + log);
    }
    size_t n = 0;
    hiprtcGetCodeSize(prog, &n);
    code->resize(n);
    hiprtcGetCode(prog, code->data());
    hiprtcDestroyProgram(&prog);
    return 0;
}

uint64_t fnv1a(const std::string& s) {
    uint64_t h = 1469598103934665603ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

std::string cache_dir() {
    const char* flag = std::getenv("MT_KERNEL_CACHE");
    if (flag && std::string(flag) == "0") return "";
    const char* dir = std::getenv("MT_KERNEL_CACHE_DIR");
    if (dir && *dir) return dir;
    const char* home = std::getenv("HOME");
    if (!home || !*home) return "";
    return std::string(home) + "/.cache/metellus_amd";
}

void mkdirs(const std::string& path) {
    std::string cur;
    for (size_t i = 0; i < path.size(); ++i) {
        cur.push_back(path[i]);
        if (path[i] == '/' || i + 1 == path.size()) mkdir(cur.c_str(), 0755);
    }
}

// A cache file holds the 8-byte length of its key, the key itself, then the
// code object.  The file name is only a hash of the key: a load compares the
// stored key with the wanted one, so a hash collision or a truncated file is
// a miss, never a wrong kernel.
bool disk_load(const std::string& file, const std::string& key, std::vector<char>* code) {
    FILE* f = std::fopen(file.c_str(), "rb");
    if (!f) return false;
    std::fseek(f, 0, SEEK_END);
    const long n = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    uint64_t klen = 0;
    bool ok = n > 8 && std::fread(&klen, sizeof(klen), 1, f) == 1 && klen == key.size() &&
              static_cast<uint64_t>(n) > 8 + klen;
    if (ok) {
        std::string stored(klen, '\0');
        ok = std::fread(&stored[0], 1, klen, f) == klen && stored == key;
    }
    if (ok) {
        code->resize(static_cast<size_t>(n) - 8 - klen);
        ok = std::fread(code->data(), 1, code->size(), f) == code->size();
    }
    std::fclose(f);
    return ok;
}

void disk_store(const std::string& dir, const std::string& file, const std::string& key,
                const std::vector<char>& code) {
    mkdirs(dir);
    std::string tmp = file + ".tmp" + std::to_string(static_cast<long>(getpid()));
    FILE* f = std::fopen(tmp.c_str(), "wb");
    if (!f) return;
    const uint64_t klen = key.size();
    bool ok = std::fwrite(&klen, sizeof(klen), 1, f) == 1 &&
              std::fwrite(key.data(), 1, key.size(), f) == key.size() &&
              std::fwrite(code.data(), 1, code.size(), f) == code.size();
    ok = (std::fclose(f) == 0) && ok;
    if (ok) std::rename(tmp.c_str(), file.c_str());
    else std::remove(tmp.c_str());
}

// The compiler's version is part of every cache key, so code objects built
// by another hiprtc are never reused.
std::string compiler_tag() {
    int major = 0, minor = 0;
    if (hiprtcVersion(&major, &minor) != HIPRTC_SUCCESS) return "hiprtc-unknown";
    return "hiprtc-" + std::to_string(major) + "." + std::to_string(minor);
}

}  // namespace

extern "C" {

const char* mt_last_error(void) { return g_error.c_str(); }

int mt_init(void) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    return init_locked(s);
}

int mt_device_count(int* count) {
    if (!count) return fail("mt_device_count: null output");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    *count = (e == hipSuccess) ? n : 0;
    return 0;
}

int mt_device_info(char* arch, size_t arch_len, int* cu_count, int* clock_khz) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (init_locked(s)) return 1;
    if (arch && arch_len) {
        std::strncpy(arch, s.arch.c_str(), arch_len - 1);
        arch[arch_len - 1] = '\0';
    }
    if (cu_count) *cu_count = s.cu_count;
    if (clock_khz) *clock_khz = s.clock_khz;
    return 0;
}

int mt_device_pci(char* bus_id, size_t bus_id_len, int* mem_clock_khz, uint64_t* total_mem) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (init_locked(s)) return 1;
    if (bus_id && bus_id_len) MT_HIP(hipDeviceGetPCIBusId(bus_id, static_cast<int>(bus_id_len), 0));
    hipDeviceProp_t prop;
    MT_HIP(hipGetDeviceProperties(&prop, 0));
    if (mem_clock_khz) *mem_clock_khz = prop.memoryClockRate;
    if (total_mem) *total_mem = static_cast<uint64_t>(prop.totalGlobalMem);
    return 0;
}

// Hand every cached device block back to the driver (stream-ordered).
static int release_dev_cache(State& s) {
    for (auto& kv : s.dev_free) MT_HIP(hipFreeAsync(kv.second, s.stream));
    s.dev_free.clear();
    s.dev_cached = 0;
    return 0;
}

int mt_alloc(size_t nbytes, uint64_t* handle) {
    if (!handle) return fail("mt_alloc: null output");
    if (nbytes == 0) return fail("create_buffer: nbytes must be > 0");
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (init_locked(s)) return 1;
    const size_t cap = dev_capacity(nbytes);
    void* p = nullptr;
    size_t got = cap;
    // The smallest cached block of at least cap bytes, wasting at most 1/8.
    auto it = s.dev_free.lower_bound(cap);
    if (it != s.dev_free.end() && it->first <= cap + cap / 8) {
        p = it->second;
        got = it->first;
        s.dev_cached -= got;
        s.dev_free.erase(it);
    } else {
        hipError_t e = hipMallocAsync(&p, cap, s.stream);
        if (e == hipErrorOutOfMemory && !s.dev_free.empty()) {
            (void)hipGetLastError();
            if (release_dev_cache(s)) return 1;
            MT_HIP(hipStreamSynchronize(s.stream));
            e = hipMallocAsync(&p, cap, s.stream);
        }
        if (e != hipSuccess) return fail(std::string("hipMallocAsync: ") + hipGetErrorString(e));
        ++s.device_allocs;
    }
    uint64_t h = s.next_buffer++;
    s.buffers.emplace(h, Buffer{p, nbytes, got});
    *handle = h;
    return 0;
}

int mt_trim(void) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (!s.ready) return 0;
    if (release_dev_cache(s)) return 1;
    MT_HIP(hipStreamSynchronize(s.stream));
    return 0;
}

int mt_alloc_stats(uint64_t* device_allocs, uint64_t* host_allocs, uint64_t* live_buffers,
                   size_t* workspace_bytes) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (device_allocs) *device_allocs = s.device_allocs;
    if (host_allocs) *host_allocs = s.host_allocs;
    if (live_buffers) *live_buffers = s.buffers.size();
    if (workspace_bytes) *workspace_bytes = s.ws_bytes;
    return 0;
}

int mt_cache_info(size_t* cached_bytes, size_t* cached_blocks) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (cached_bytes) *cached_bytes = s.dev_cached;
    if (cached_blocks) *cached_blocks = s.dev_free.size();
    return 0;
}

int mt_free(uint64_t handle, int* existed) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (handle != 0 && handle == s.ws_handle) return fail("mt_free: the workspace belongs to the shim");
    auto it = s.buffers.find(handle);
    if (it == s.buffers.end()) {
        if (existed) *existed = 0;
        return 0;
    }
    const Buffer b = it->second;
    s.buffers.erase(it);
    if (existed) *existed = 1;
    // Kept for reuse (the device block cache) while the cache has room;
    // otherwise returned, stream-ordered: kernels already queued that read
    // the buffer finish first either way.
    if (s.dev_cached + b.cap <= s.dev_cache_limit) {
        s.dev_free.emplace(b.cap, b.ptr);
        s.dev_cached += b.cap;
        return 0;
    }
    MT_HIP(hipFreeAsync(b.ptr, s.stream));
    return 0;
}

static int lookup(State& s, uint64_t handle, Buffer* out) {
    auto it = s.buffers.find(handle);
    if (it == s.buffers.end()) return fail("Unknown buffer handle: " + std::to_string(handle));
    *out = it->second;
    return 0;
}

int mt_size(uint64_t handle, size_t* nbytes) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    Buffer b;
    if (lookup(s, handle, &b)) return 1;
    if (nbytes) *nbytes = b.nbytes;
    return 0;
}

int mt_device_ptr(uint64_t handle, uint64_t* address) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    Buffer b;
    if (lookup(s, handle, &b)) return 1;
    if (address) *address = reinterpret_cast<uint64_t>(b.ptr);
    return 0;
}

int mt_write(uint64_t handle, const void* src, size_t nbytes) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    Buffer b;
    if (lookup(s, handle, &b)) return 1;
    if (nbytes > b.nbytes) return fail("write_buffer: source larger than buffer");
    if (nbytes == 0) return 0;
    if (!src) return fail("write_buffer: null source");
    if (nbytes >= kStageMin && !is_pinned(src))
        return staged_upload(s, static_cast<char*>(b.ptr), static_cast<const char*>(src), nbytes);
    MT_HIP(hipMemcpyAsync(b.ptr, src, nbytes, hipMemcpyHostToDevice, s.stream));
    MT_HIP(hipStreamSynchronize(s.stream));
    return 0;
}

int mt_read(uint64_t handle, void* dst, size_t nbytes) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    Buffer b;
    if (lookup(s, handle, &b)) return 1;
    if (nbytes > b.nbytes) return fail("read_buffer: destination larger than buffer");
    if (nbytes == 0) return 0;
    if (!dst) return fail("read_buffer: null destination");
    if (nbytes >= kStageMin && !is_pinned(dst))
        return staged_download(s, static_cast<char*>(dst), static_cast<const char*>(b.ptr), nbytes);
    MT_HIP(hipMemcpyAsync(dst, b.ptr, nbytes, hipMemcpyDeviceToHost, s.stream));
    MT_HIP(hipStreamSynchronize(s.stream));
    return 0;
}

int mt_host_alloc(size_t nbytes, void** ptr) {
    if (!ptr) return fail("mt_host_alloc: null output");
    if (nbytes == 0) return fail("mt_host_alloc: nbytes must be > 0");
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (init_locked(s)) return 1;
    const size_t want = (nbytes + kHostGranule - 1) / kHostGranule * kHostGranule;
    // Reuse the smallest cached block that fits without wasting more than half.
    auto it = s.host_free.lower_bound(want);
    if (it != s.host_free.end() && it->first <= 2 * want) {
        *ptr = it->second;
        s.host_cached -= it->first;
        s.host_free.erase(it);
        return 0;
    }
    void* p = nullptr;
    MT_HIP(hipHostMalloc(&p, want, hipHostMallocDefault));
    ++s.host_allocs;
    s.host_cap.emplace(p, want);
    *ptr = p;
    return 0;
}

int mt_host_free(void* ptr) {
    if (!ptr) return 0;
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    auto it = s.host_cap.find(ptr);
    if (it == s.host_cap.end()) return fail("mt_host_free: pointer was not returned by mt_host_alloc");
    const size_t cap = it->second;
    if (s.host_cached + cap <= kHostCacheLimit) {
        s.host_free.emplace(cap, ptr);
        s.host_cached += cap;
        return 0;
    }
    s.host_cap.erase(it);
    MT_HIP(hipHostFree(ptr));
    return 0;
}

int mt_fill(uint64_t handle, uint8_t value) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    Buffer b;
    if (lookup(s, handle, &b)) return 1;
    MT_HIP(hipMemsetAsync(b.ptr, value, b.nbytes, s.stream));
    return 0;
}

int mt_compile_only(const char* source, const char* options, const char* target, size_t* code_size) {
    if (!source) return fail("mt_compile_only: null source");
    std::vector<char> code;
    std::string t = (target && *target) ? target : "gfx950";
    if (rtc_compile(source, full_options(t, options), &code)) return 1;
    if (code_size) *code_size = code.size();
    return 0;
}

int mt_compile(const char* source, const char* function_name, const char* options, uint64_t* kernel) {
    if (!source || !function_name || !kernel) return fail("mt_compile: null argument");
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (init_locked(s)) return 1;
    std::vector<std::string> opts = full_options(s.arch, options);
    std::string key;
    key.reserve(std::strlen(source) + 256);
    key.append(source).push_back('\0');
    key.append(function_name).push_back('\0');
    for (auto& o : opts) key.append(o).push_back(' ');
    static const std::string tag = compiler_tag();
    key.append(tag);
    auto hit = s.by_key.find(key);
    if (hit != s.by_key.end()) {
        ++s.hits;
        *kernel = hit->second;
        return 0;
    }
    std::vector<char> code;
    std::string dir = cache_dir();
    char name[32];
    std::snprintf(name, sizeof(name), "%016llx.co", static_cast<unsigned long long>(fnv1a(key)));
    std::string file = dir.empty() ? "" : dir + "/" + name;
    if (!file.empty() && disk_load(file, key, &code)) {
        ++s.hits;
    } else {
        if (rtc_compile(source, opts, &code)) return 1;
        ++s.compiled;
        if (!file.empty()) disk_store(dir, file, key, code);
    }
    Kernel k{};
    MT_HIP(hipModuleLoadData(&k.module, code.data()));
    hipError_t e = hipModuleGetFunction(&k.function, k.module, function_name);
    if (e != hipSuccess) {
        (void)hipModuleUnload(k.module);
        return fail(std::string("kernel function was not found: ") + function_name + " (" +
                    hipGetErrorString(e) + ")");
    }
    s.kernels.push_back(k);
    uint64_t h = s.kernels.size();
    s.by_key.emplace(std::move(key), h);
    *kernel = h;
    return 0;
}

int mt_launch(uint64_t kernel, const uint64_t* buffers, int nbuf, const uint32_t* dims, int ndims,
              int dims_slot, const uint32_t* grid, const uint32_t* block, int timed, float* ms) {
    if (!grid || !block) return fail("mt_launch: grid and block are required");
    if (ndims < 0 || ndims > kMaxDims) return fail("mt_launch: at most 16 dims");
    if (nbuf < 0 || dims_slot < 0 || dims_slot > nbuf) return fail("mt_launch: bad dims slot");
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (init_locked(s)) return 1;
    if (kernel == 0 || kernel > s.kernels.size()) return fail("mt_launch: unknown kernel handle");
    for (int i = 0; i < 3; ++i) {
        if (grid[i] == 0 || block[i] == 0) return fail("mt_launch: zero grid or block extent");
    }
    if (static_cast<uint64_t>(block[0]) * block[1] * block[2] > 1024)
        return fail("mt_launch: more than 1024 lanes per workgroup");
    std::vector<void*> ptrs(static_cast<size_t>(nbuf));
    for (int i = 0; i < nbuf; ++i) {
        Buffer b;
        if (lookup(s, buffers[i], &b)) return 1;
        ptrs[i] = b.ptr;
    }
    DimsArg d{};
    for (int i = 0; i < ndims; ++i) d.v[i] = dims[i];
    std::vector<void*> params;
    params.reserve(static_cast<size_t>(nbuf) + 1);
    for (int i = 0; i <= nbuf; ++i) {
        if (i == dims_slot) params.push_back(&d);
        if (i < nbuf) params.push_back(&ptrs[i]);
    }
    const Kernel& k = s.kernels[kernel - 1];
    if (timed) MT_HIP(hipEventRecord(s.ev_start, s.stream));
    MT_HIP(hipModuleLaunchKernel(k.function, grid[0], grid[1], grid[2], block[0], block[1], block[2], 0,
                                 s.stream, params.data(), nullptr));
    if (timed) {
        MT_HIP(hipEventRecord(s.ev_stop, s.stream));
        MT_HIP(hipEventSynchronize(s.ev_stop));
        float t = 0.f;
        MT_HIP(hipEventElapsedTime(&t, s.ev_start, s.ev_stop));
        if (ms) *ms = t;
    }
    return 0;
}

int mt_launch_noalloc(uint64_t kernel, const uint64_t* buffers, int nbuf, const uint32_t* dims, int ndims,
                      int dims_slot, const uint32_t* grid, const uint32_t* block, size_t scratch_bytes,
                      uint32_t* error) {
    if (!grid || !block) return fail("mt_launch_noalloc: grid and block are required");
    if (ndims < 0 || ndims > kMaxDims) return fail("mt_launch_noalloc: at most 16 dims");
    if (nbuf < 0 || nbuf > kMaxLaunchBuffers) return fail("mt_launch_noalloc: at most 64 buffers");
    if (dims_slot < 0 || dims_slot > nbuf) return fail("mt_launch_noalloc: bad dims slot");
    if (scratch_bytes > kScratchBytes)
        return fail("mt_launch_noalloc: the kernel needs " + std::to_string(scratch_bytes) +
                    " bytes of scratch; the static scratch holds " + std::to_string(kScratchBytes));
    if (scratch_bytes != 0 && scratch_bytes < kWsHeadBytes)
        return fail("mt_launch_noalloc: a scratch request covers at least the 4096-byte flag head");
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    // Initialisation creates the stream and events; this entry point does
    // not do it on a caller's behalf.
    if (!s.ready) return fail("mt_launch_noalloc: call mt_init first");
    if (kernel == 0 || kernel > s.kernels.size()) return fail("mt_launch_noalloc: unknown kernel handle");
    for (int i = 0; i < 3; ++i) {
        if (grid[i] == 0 || block[i] == 0) return fail("mt_launch_noalloc: zero grid or block extent");
    }
    if (static_cast<uint64_t>(block[0]) * block[1] * block[2] > 1024)
        return fail("mt_launch_noalloc: more than 1024 lanes per workgroup");
    void* ptrs[kMaxLaunchBuffers];
    for (int i = 0; i < nbuf; ++i) {
        Buffer b;
        if (lookup(s, buffers[i], &b)) return 1;
        ptrs[i] = b.ptr;
    }
    DimsArg d{};
    for (int i = 0; i < ndims; ++i) d.v[i] = dims[i];
    void* params[kMaxLaunchBuffers + 2];
    int np = 0;
    for (int i = 0; i <= nbuf; ++i) {
        if (i == dims_slot) params[np++] = &d;
        if (i < nbuf) params[np++] = &ptrs[i];
    }
    void* ws = s.scratch_ptr[0];
    if (scratch_bytes != 0) {
        // Flags and the error word start at 0 on every call: a previous
        // launch that gave up waiting may have left flags raised.
        constexpr uint32_t words = kWsHeadBytes / sizeof(uint32_t);
        hipLaunchKernelGGL(mt_clear_words, dim3(words / 256), dim3(256), 0, s.stream, static_cast<uint32_t*>(ws),
                           words);
        MT_HIP(hipGetLastError());
        params[np++] = &ws;
    }
    const Kernel& k = s.kernels[kernel - 1];
    MT_HIP(hipModuleLaunchKernel(k.function, grid[0], grid[1], grid[2], block[0], block[1], block[2], 0,
                                 s.stream, params, nullptr));
    if (error) {
        *error = 0;
        if (scratch_bytes != 0)
            MT_HIP(hipMemcpyAsync(error, static_cast<char*>(ws) + kWsErrorOffset, sizeof(uint32_t),
                                  hipMemcpyDeviceToHost, s.stream));
        MT_HIP(hipStreamSynchronize(s.stream));
    }
    return 0;
}

int mt_workspace(size_t nbytes, uint64_t* handle) {
    if (!handle) return fail("mt_workspace: null output");
    if (nbytes < kWsHeadBytes) return fail("mt_workspace: a workspace holds at least its 4096-byte head");
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (init_locked(s)) return 1;
    if (nbytes > s.ws_bytes) {
        if (s.ws_handle) {
            // Stream-ordered: kernels already queued on the old one finish first.
            MT_HIP(hipFreeAsync(s.buffers[s.ws_handle].ptr, s.stream));
            s.buffers.erase(s.ws_handle);
            s.ws_handle = 0;
            s.ws_bytes = 0;
        }
        void* p = nullptr;
        MT_HIP(hipMallocAsync(&p, nbytes, s.stream));
        ++s.device_allocs;
        MT_HIP(hipMemsetAsync(p, 0, kWsHeadBytes, s.stream));  // flags and error word start at 0
        s.ws_handle = s.next_buffer++;
        s.buffers.emplace(s.ws_handle, Buffer{p, nbytes, nbytes});
        s.ws_bytes = nbytes;
    }
    *handle = s.ws_handle;
    return 0;
}

int mt_workspace_check(uint32_t* error) {
    if (!error) return fail("mt_workspace_check: null output");
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    *error = 0;
    if (!s.ws_handle) return 0;
    char* p = static_cast<char*>(s.buffers[s.ws_handle].ptr);
    uint32_t word = 0;
    MT_HIP(hipMemcpyAsync(&word, p + kWsErrorOffset, sizeof(word), hipMemcpyDeviceToHost, s.stream));
    MT_HIP(hipStreamSynchronize(s.stream));
    if (word != 0) {
        // A wait gave up: its flags may be stale, so start the next launch clean.
        MT_HIP(hipMemsetAsync(p, 0, kWsHeadBytes, s.stream));
        MT_HIP(hipStreamSynchronize(s.stream));
    }
    *error = word;
    return 0;
}

int mt_mark(int slot) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (init_locked(s)) return 1;
    if (slot < 0 || slot >= 16) return fail("mt_mark: slot must be in [0, 16)");
    MT_HIP(hipEventRecord(s.marks[slot], s.stream));
    return 0;
}

int mt_mark_elapsed(int from, int to, float* ms) {
    if (!ms) return fail("mt_mark_elapsed: null output");
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (init_locked(s)) return 1;
    if (from < 0 || from >= 16 || to < 0 || to >= 16) return fail("mt_mark_elapsed: slots must be in [0, 16)");
    MT_HIP(hipEventSynchronize(s.marks[to]));
    MT_HIP(hipEventElapsedTime(ms, s.marks[from], s.marks[to]));
    return 0;
}

int mt_sync(void) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (init_locked(s)) return 1;
    MT_HIP(hipStreamSynchronize(s.stream));
    return 0;
}

int mt_cache_stats(uint64_t* compiled, uint64_t* hits) {
    State& s = state();
    std::lock_guard<std::mutex> lock(s.mu);
    if (compiled) *compiled = s.compiled;
    if (hits) *hits = s.hits;
    return 0;
}

}  // extern "C"
