// vnpu_internal.hpp - private object model of the MI355X vnpu backend.
//
// The reference runtime keeps its opaque objects in src/internal.h:618-725
// (device with a CPU thread pool, stream with a worker thread, event with a
// condition variable, host buffers).  Here the same handles wrap HIP objects:
//   vnpu_device  -> one HIP device (ordinal), counters, trace, MMIO registers
//   vnpu_stream  -> one hipStream_t plus a growable device workspace
//   vnpu_event   -> one hipEvent_t recorded at the end of a submitted batch
//   vnpu_buffer  -> one hipMalloc allocation in HBM
//   vnpu_packed_weights -> int8 weights in HBM in the MFMA fragment layout
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "vnpu.h"

namespace vnpu {

// A HIP failure inside a command becomes a command failure (sticky stream
// error), never an abort; no C++ exception crosses the C ABI.
struct HipError : std::runtime_error {
    explicit HipError(const std::string &s) : std::runtime_error(s) {}
};

#define VNPU_HIP(expr)                                                           \
    do {                                                                         \
        hipError_t _e = (expr);                                                  \
        if (_e != hipSuccess)                                                    \
            throw ::vnpu::HipError(std::string(#expr) + ": " + hipGetErrorString(_e)); \
    } while (0)

struct ArgError : std::runtime_error {
    explicit ArgError(const char *s) : std::runtime_error(s) {}
};

bool debug_enabled();
void debug_log(const char *fmt, ...);

template <typename F>
inline vnpu_status_t guard(F &&fn) noexcept
{
    try {
        return fn();
    } catch (const std::bad_alloc &) {
        return VNPU_ERR_OUT_OF_MEMORY;
    } catch (const std::exception &e) {
        debug_log("exception: %s", e.what());
        return VNPU_ERR_INTERNAL;
    } catch (...) {
        return VNPU_ERR_INTERNAL;
    }
}

// One traced command: host-side accounting plus a pair of hipEvents on the
// command's stream (resolved lazily when a summary is requested).
struct TraceRecord {
    uint32_t opcode = 0;
    uint32_t unit = 0;
    uint64_t id = 0;
    uint64_t bytes_read = 0;
    uint64_t bytes_written = 0;
    uint64_t flops = 0;
    uint64_t host_ns = 0;
    uint64_t gpu_ns = 0;
    uint64_t gpu_start_ns = 0;   // GPU start relative to the trace epoch
    bool resolved = false;
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};

struct TraceState {
    std::atomic<bool> enabled{false};
    std::mutex mutex;
    std::vector<TraceRecord> records;
    hipEvent_t epoch = nullptr;   // recorded before the first traced command
    std::string trace_file;
    void reset();
    void resolve();  // waits for and converts pending hipEvent pairs
};

}  // namespace vnpu

struct vnpu_event {
    std::mutex mutex;
    hipEvent_t hip = nullptr;      // recorded at the end of the last batch
    int hip_device = -1;
    bool submitted = false;        // a batch carrying this event was submitted
    bool host_signaled = false;    // completed without GPU work (empty batch)
    vnpu_status_t status = VNPU_OK;
    uint64_t command_count = 0;
};

struct vnpu_buffer {
    vnpu_device_t *device = nullptr;
    void *dev_ptr = nullptr;
    uint64_t bytes = 0;
    uint64_t handle = 0;
};

struct vnpu_packed_weights {
    vnpu_device_t *device = nullptr;
    uint32_t K = 0, N = 0;
    uint32_t Kp = 0;               // K rounded up to 64
    uint32_t Np = 0;               // N rounded up to 16
    int8_t *frag = nullptr;        // HBM, [Np/16][Kp/64][4][16][16] fragment layout
    float *scales_dev = nullptr;   // HBM [Np], padding = 1
    uint64_t frag_bytes = 0;
    // Nonzero 64 x 64 tiles (k::tile_lists): HBM [groups][Kp/64] k-block
    // lists and [groups] counts, groups = ceil(Np / 64); nz_tiles in total.
    uint32_t *nz_list = nullptr;
    uint32_t *nz_count = nullptr;
    uint64_t nz_tiles = 0;
    std::vector<float> scales;     // host copies for vnpu_packed_weights_info
    std::vector<int32_t> column_sums;
};

struct vnpu_stream {
    vnpu_device_t *device = nullptr;
    int priority = 0;
    hipStream_t hip = nullptr;
    std::mutex mutex;              // one submitter at a time per stream
    std::atomic<uint32_t> last_error{0};
    std::atomic<uint64_t> pending{0};
    void *workspace = nullptr;
    size_t workspace_bytes = 0;
    // Error word of the kernels on this stream whose bounded waits may give
    // up (pinned, host-coherent: err_host on the host, err_dev in kernels);
    // nonzero at a sync = a launch since the last sync computed garbage.
    uint32_t *err_host = nullptr;
    uint32_t *err_dev = nullptr;
    // Device copies of host-pointer operands: one grow-only arena reused by
    // every staged command (each staged command synchronizes before it
    // returns, so the next one may overwrite it).  Guarded by mutex.
    void *staging = nullptr;
    size_t staging_bytes = 0;
    // The cull map and kernel-tile states of a MATMUL_F32 whose tile mask is
    // in device memory, built on the GPU in stream order (grow-only).
    void *cull_scratch = nullptr;
    size_t cull_scratch_bytes = 0;
    void *ensure_cull_scratch(size_t bytes);
    void *ensure_workspace(size_t bytes);
    // GPU time of submitted work by busy periods: a timing event is recorded
    // before the first batch after a synchronization and another when the
    // period closes (stream sync, stream destruction, every 256 batches);
    // closed pairs are folded into the device's kernel time once complete.
    // Every event record on a stream costs the next kernel ~3 us of start
    // latency, so a pair per batch would tax every batch.  Guarded by mutex.
    std::vector<std::pair<hipEvent_t, hipEvent_t>> batch_timing;
    std::vector<hipEvent_t> event_pool;
    hipEvent_t period_start = nullptr;
    uint32_t period_batches = 0;
    hipEvent_t acquire_event();
    void open_period();
    void close_period();
    void resolve_timing(bool wait_all);   // adds finished pairs to kernel_ns
};

struct vnpu_device {
    vnpu_config_t config{};
    vnpu_device_info_t info{};
    int hip_device = 0;
    uint32_t cu_count = 0;
    vnpu::TraceState trace;
    std::atomic<uint32_t> regs[VNPU_REG_COUNT];
    std::atomic<uint64_t> commands_submitted{0};
    std::atomic<uint64_t> commands_completed{0};
    std::atomic<uint64_t> kernel_ns{0};
    std::atomic<uint64_t> dispatch_ns{0};
    std::atomic<uint64_t> memory_ns{0};
    std::atomic<uint64_t> sync_ns{0};
    std::atomic<uint64_t> bytes_read{0};
    std::atomic<uint64_t> bytes_written{0};
    std::atomic<uint64_t> flops{0};
    std::atomic<uint64_t> tiles_dispatched{0};
    std::atomic<uint64_t> tiles_culled{0};
    std::atomic<uint64_t> dma_bytes{0};
    std::atomic<uint64_t> interrupts{0};
    std::atomic<uint32_t> busy{0};
    std::atomic<uint32_t> error{0};
    std::atomic<uint32_t> active_workers{0};
    std::atomic<uint32_t> last_opcode{0};
    std::atomic<uint32_t> tile_m{0}, tile_k{0}, tile_n{0};
    // GEMM kernels forced by tile triples, one choice per dtype: set together
    // by vnpu_device_set_tiles, but vnpu_autotune_gemm writes only the choice
    // of the dtype it tuned.  0 = automatic.
    std::atomic<uint32_t> i8_variant{0};   // int8 GEMM kernel (gemm_i8_variant_for_tiles)
    std::atomic<uint32_t> f32_depth{0};    // f32 K depth per workgroup (split-K)
    bool reference_order = true;           // attention bit-exact (off: VNPU_CONFIG_HIGH_THROUGHPUT)
    uint32_t ws_max_spin = 0;              // bound of the f32 GEMM's flag waits (0: kernel default)
    // Culled tiles counted on the GPU (MATMUL_F32 with a device-resident tile
    // mask); folded into the status when read.  Allocated on first use.
    unsigned long long *culled_dev = nullptr;
    std::mutex culled_mutex;
    std::vector<vnpu_stream_t *> streams;
    std::mutex stream_mutex;
    vnpu_interrupt_cb_t irq_cb = nullptr;
    void *irq_user = nullptr;
    std::mutex irq_mutex;
    std::string name;
    void raise_irq(uint32_t bits);
};

namespace vnpu {

// Accounting for one command, mirroring the reference's per-op byte/flop
// model (src/core/scheduler.cpp execute_* functions).
struct ExecStats {
    uint64_t bytes_read = 0;
    uint64_t bytes_written = 0;
    uint64_t flops = 0;
    uint64_t dma_bytes = 0;
    uint64_t tiles_dispatched = 0;
    uint64_t tiles_culled = 0;
    uint32_t unit = 0;
};

// Two independent MATMUL_I8 commands in one grid; false: run them one by one.
bool try_execute_pair(vnpu_device_t *dev, vnpu_stream_t *s, const vnpu_command_t &c0,
                      const vnpu_command_t &c1, uint32_t flags, ExecStats &st0, ExecStats &st1);
// MATMUL_I8 (M <= 8) then an ADD_F32 of its output in one GEMV launch;
// false: run them one by one.
bool try_execute_matmul_add(vnpu_device_t *dev, vnpu_stream_t *s, const vnpu_command_t &c0,
                            const vnpu_command_t &c1, uint32_t flags, ExecStats &st0, ExecStats &st1);
// A row chain at the head of c[0..n): ADD -> RMSNORM [-> QUANTIZE_I8 per row],
// RMSNORM -> QUANTIZE_I8 or SWIGLU -> QUANTIZE_I8 over the same rows, device
// buffers only, run as one kernel.  Returns the number of commands executed
// (0: none, run them one by one); *matched is set before the launch so a
// caller that catches a HipError knows how many commands it covered.  st[]
// holds one entry per executed command.
uint32_t try_execute_chain(vnpu_stream_t *s, const vnpu_command_t *c, uint64_t n,
                           uint32_t *matched, ExecStats *st);
// Executes one command on the stream (enqueue only).  Throws ArgError for
// invalid arguments and HipError for runtime failures.
void execute_command(vnpu_device_t *dev, vnpu_stream_t *s, const vnpu_command_t &cmd,
                     uint32_t batch_flags, ExecStats &st);

// ATTENTION_F32 on device-resident tensors with the device scratch of
// attention.hip instead of the stream workspace: enqueues only, allocates
// nothing.  Throws ArgError for invalid arguments, host pointers or a
// scratch need above k::kAttnScratchBytes.
void enqueue_attention_noalloc(vnpu_stream_t *s, const vnpu_attention_f32_args_t &a, ExecStats &st);
// Pack int8 weights (synchronous); B and tile_mask may be host or device
// pointers.  A non-null tile_mask ([ceil(K/64)][mask_ld] bytes; mask_ld 0 =
// ceil(N/64)) packs the 64 x 64 tiles whose byte is zero as zeros.
vnpu_packed_weights_t *pack_weights(vnpu_device_t *dev, const int8_t *B, const float *scales,
                                    uint32_t K, uint32_t N, uint32_t ldb, uint32_t trans_b,
                                    const uint8_t *tile_mask = nullptr, uint32_t mask_ld = 0);
void destroy_packed(vnpu_packed_weights_t *w);

bool is_device_pointer(const void *p);
// Ranges this library allocated in HBM: classified without a HIP query.
void register_device_range(const void *p, size_t bytes);
void unregister_device_range(const void *p);

}  // namespace vnpu
