// runtime.cpp - the vnpu C ABI on HIP (device, stream, event, buffer, trace).
//
// Replaces the reference runtime (src/core/runtime.cpp) and backend table
// (src/core/backend.cpp).  The mapping:
//   vnpu_device_create   -> a HIP device ordinal (VNPU_HIP_DEVICE, default 0)
//   vnpu_stream_*        -> hipStream_t at default priority; submit enqueues
//                           every command of the batch in order on the caller
//                           thread, sync is hipStreamSynchronize
//   vnpu_event_*         -> hipEvent_t recorded after the batch
//   vnpu_buffer_*        -> hipMalloc'd HBM (zero filled, as the reference)
//   Sherlock trace       -> hipEvent pairs around each command
// Error behaviour follows the reference: submit only rejects a null stream or
// an oversized batch; a failing command marks the batch event with its
// status and makes every later sync of that stream return
// VNPU_ERR_DEVICE_ERROR (sticky, runtime.cpp:1248-1254, 1281-1289).
#include "vnpu_internal.hpp"
#include "vnpu_backend.h"
#include "kernels.hpp"

#include <algorithm>
#include <vector>
#include <limits>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstring>
#include <fstream>
#include <sstream>
#include <thread>

namespace vnpu {

void release_device_tables(vnpu_device_t *dev);

bool debug_enabled()
{
    static const bool on = std::getenv("VNPU_DEBUG") != nullptr;
    return on;
}

void debug_log(const char *fmt, ...)
{
    if (!debug_enabled()) return;
    va_list ap;
    va_start(ap, fmt);
    std::fprintf(stderr, "[vnpu-mi355x] ");
    std::vfprintf(stderr, fmt, ap);
    std::fputc('\n', stderr);
    va_end(ap);
}

static uint64_t now_ns()
{
    return static_cast<uint64_t>(std::chrono::duration_cast<std::chrono::nanoseconds>(
                                     std::chrono::steady_clock::now().time_since_epoch())
                                     .count());
}

void TraceState::reset()
{
    std::lock_guard<std::mutex> lock(mutex);
    for (auto &r : records) {
        if (r.start) (void)hipEventDestroy(r.start);
        if (r.stop) (void)hipEventDestroy(r.stop);
    }
    records.clear();
    if (epoch) (void)hipEventDestroy(epoch);
    epoch = nullptr;
}

void TraceState::resolve()
{
    std::lock_guard<std::mutex> lock(mutex);
    for (auto &r : records) {
        if (r.resolved) continue;
        float ms = 0.0f, ms0 = 0.0f;
        if (r.start && r.stop && hipEventSynchronize(r.stop) == hipSuccess &&
            hipEventElapsedTime(&ms, r.start, r.stop) == hipSuccess)
            r.gpu_ns = static_cast<uint64_t>(static_cast<double>(ms) * 1e6);
        else
            (void)hipGetLastError();
        if (epoch && r.start && hipEventElapsedTime(&ms0, epoch, r.start) == hipSuccess)
            r.gpu_start_ns = ms0 > 0.0f ? static_cast<uint64_t>(static_cast<double>(ms0) * 1e6) : 0;
        else
            (void)hipGetLastError();
        if (r.start) (void)hipEventDestroy(r.start);
        if (r.stop) (void)hipEventDestroy(r.stop);
        r.start = r.stop = nullptr;
        r.resolved = true;
    }
}

static uint32_t trace_category(uint32_t opcode)
{
    if (opcode == VNPU_OP_COPY || opcode == VNPU_OP_MEMSET || opcode == VNPU_OP_PACK_WEIGHTS_I8)
        return 1;  // memory
    if (opcode == VNPU_OP_BARRIER || opcode == VNPU_OP_NOP) return 2;  // sync
    return 0;  // compute
}

}  // namespace vnpu

using namespace vnpu;

void *vnpu_stream::ensure_workspace(size_t bytes)
{
    if (bytes == 0) return workspace;
    if (bytes <= workspace_bytes) return workspace;
    if (workspace) {
        VNPU_HIP(hipStreamSynchronize(hip));
        VNPU_HIP(hipFree(workspace));
        workspace = nullptr;
        workspace_bytes = 0;
    }
    size_t want = std::max<size_t>(bytes, 1u << 20);
    VNPU_HIP(hipMalloc(&workspace, want));
    workspace_bytes = want;
    return workspace;
}

void *vnpu_stream::ensure_cull_scratch(size_t bytes)
{
    if (bytes <= cull_scratch_bytes) return cull_scratch;
    if (cull_scratch) {
        VNPU_HIP(hipStreamSynchronize(hip));
        VNPU_HIP(hipFree(cull_scratch));
        cull_scratch = nullptr;
        cull_scratch_bytes = 0;
    }
    const size_t want = std::max<size_t>(bytes, 64u << 10);
    VNPU_HIP(hipMalloc(&cull_scratch, want));
    cull_scratch_bytes = want;
    return cull_scratch;
}

// Events that only time GPU work: no system-scope fence when they complete
// (the default event writes back and invalidates the caches, which costs
// several microseconds per record and slows the kernels that follow).
static hipError_t create_timing_event(hipEvent_t *e)
{
    return hipEventCreateWithFlags(e, hipEventDisableSystemFence);
}

hipEvent_t vnpu_stream::acquire_event()
{
    if (!event_pool.empty()) {
        hipEvent_t e = event_pool.back();
        event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (create_timing_event(&e) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return e;
}

void vnpu_stream::open_period()
{
    if (period_start) return;
    period_start = acquire_event();
    if (period_start) (void)hipEventRecord(period_start, hip);
    period_batches = 0;
}

void vnpu_stream::close_period()
{
    if (!period_start) return;
    hipEvent_t stop = acquire_event();
    if (stop) {
        (void)hipEventRecord(stop, hip);
        batch_timing.emplace_back(period_start, stop);
    } else {
        event_pool.push_back(period_start);
    }
    period_start = nullptr;
    period_batches = 0;
}

void vnpu_stream::resolve_timing(bool wait_all)
{
    size_t keep = 0;
    for (size_t i = 0; i < batch_timing.size(); ++i) {
        auto &pr = batch_timing[i];
        if (!wait_all && hipEventQuery(pr.second) != hipSuccess) {
            (void)hipGetLastError();
            batch_timing[keep++] = pr;
            continue;
        }
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, pr.first, pr.second) == hipSuccess && ms > 0.0f)
            device->kernel_ns.fetch_add(static_cast<uint64_t>(static_cast<double>(ms) * 1e6));
        else
            (void)hipGetLastError();
        event_pool.push_back(pr.first);
        event_pool.push_back(pr.second);
    }
    batch_timing.resize(keep);
}

void vnpu_device::raise_irq(uint32_t bits)
{
    const uint32_t old = regs[VNPU_REG_IRQ_STATUS / 4].fetch_or(bits);
    const uint32_t mask = regs[VNPU_REG_IRQ_MASK / 4].load();
    if ((old & bits) == 0 && (mask & bits)) {
        interrupts.fetch_add(1);
        vnpu_interrupt_cb_t cb;
        void *user;
        {
            std::lock_guard<std::mutex> lock(irq_mutex);
            cb = irq_cb;
            user = irq_user;
        }
        if (cb) cb(this, bits, user);
    }
}

extern "C" {

// ---------------------------------------------------------------------------
// Small helpers (reference runtime.cpp:636-815)
// ---------------------------------------------------------------------------

VNPU_API void VNPU_CALL vnpu_config_init(vnpu_config_t *config)
{
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->abi_version = VNPU_ABI_VERSION;
    if (const char *t = std::getenv("VNPU_THREADS")) config->num_threads = static_cast<uint32_t>(std::atoi(t));
    if (const char *t = std::getenv("VNPU_TRACE"))
        if (std::atoi(t)) config->flags |= VNPU_CONFIG_TRACE;
    if (const char *f = std::getenv("VNPU_TRACE_FILE")) config->trace_file = f;
}

VNPU_API const char *VNPU_CALL vnpu_status_string(vnpu_status_t status)
{
    switch (status) {
    case VNPU_OK: return "OK";
    case VNPU_ERR_INVALID_ARGUMENT: return "invalid argument";
    case VNPU_ERR_OUT_OF_MEMORY: return "out of memory";
    case VNPU_ERR_UNSUPPORTED: return "unsupported";
    case VNPU_ERR_INVALID_COMMAND: return "invalid command";
    case VNPU_ERR_DEVICE_BUSY: return "device busy";
    case VNPU_ERR_DEVICE_ERROR: return "device error";
    case VNPU_ERR_TIMEOUT: return "timeout";
    case VNPU_ERR_NETWORK: return "network error";
    case VNPU_ERR_AUTH: return "authentication error";
    case VNPU_ERR_PROTOCOL: return "protocol error";
    case VNPU_ERR_NOT_FOUND: return "not found";
    case VNPU_ERR_IO: return "I/O error";
    default: return "internal error";
    }
}

VNPU_API const char *VNPU_CALL vnpu_version_string(void) { return "vnpu 1.0.0 (MI355X gfx950)"; }

VNPU_API uint32_t VNPU_CALL vnpu_abi_version(void) { return VNPU_ABI_VERSION; }

VNPU_API const char *VNPU_CALL vnpu_opcode_name(uint32_t opcode)
{
    static const char *names[] = {"NOP", "MATMUL_F32", "MATMUL_I8", "RMSNORM_F32", "SOFTMAX_F32",
                                  "ROPE_F32", "SWIGLU_F32", "GELU_F32", "ADD_F32", "MUL_F32",
                                  "ATTENTION_F32", "QUANTIZE_I8", "PACK_WEIGHTS_I8",
                                  "MTP_HEAD_F32", "COPY", "MEMSET", "BARRIER"};
    return opcode < sizeof(names) / sizeof(names[0]) ? names[opcode] : "UNKNOWN";
}

VNPU_API const char *VNPU_CALL vnpu_unit_name(uint32_t unit)
{
    switch (unit) {
    case VNPU_UNIT_AUTO: return "AUTO";
    case VNPU_UNIT_VOODOO: return "VOODOO";
    case VNPU_UNIT_WILDCAT: return "WILDCAT";
    case VNPU_UNIT_CELL: return "CELL";
    case VNPU_UNIT_GPU: return "GPU";
    default: return "UNKNOWN";
    }
}

// bf16: round to nearest even on the top 16 bits (reference runtime.cpp:730-736).
VNPU_API uint16_t VNPU_CALL vnpu_float_to_bf16(float value)
{
    uint32_t u;
    std::memcpy(&u, &value, 4);
    return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

VNPU_API float VNPU_CALL vnpu_bf16_to_float(uint16_t value)
{
    const uint32_t u = static_cast<uint32_t>(value) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// f16 conversions with the reference's rounding (runtime.cpp:746-785):
// add half an ulp of the 13 dropped bits, then truncate.
VNPU_API uint16_t VNPU_CALL vnpu_float_to_f16(float value)
{
    uint32_t f;
    std::memcpy(&f, &value, 4);
    const uint32_t sign = (f >> 16) & 0x8000u;
    const int32_t e = static_cast<int32_t>((f >> 23) & 0xffu) - 112;
    uint32_t mant = f & 0x7fffffu;
    if (e <= 0) {
        if (e < -10) return static_cast<uint16_t>(sign);
        mant = (mant | 0x800000u) >> (1 - e);
        return static_cast<uint16_t>(sign | ((mant + 0x1000u) >> 13));
    }
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u | (mant ? 0x200u : 0u));
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | ((mant + 0x1000u) >> 13));
}

VNPU_API float VNPU_CALL vnpu_f16_to_float(uint16_t value)
{
    const uint32_t sign = static_cast<uint32_t>(value & 0x8000u) << 16;
    uint32_t e = (value >> 10) & 0x1fu;
    uint32_t mant = value & 0x3ffu;
    uint32_t f;
    if (e == 0) {
        if (mant == 0) {
            f = sign;
        } else {
            e = 113;
            while (!(mant & 0x400u)) {
                mant <<= 1;
                --e;
            }
            f = sign | (e << 23) | ((mant & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        f = sign | 0x7f800000u | (mant << 13);
    } else {
        f = sign | ((e + 112) << 23) | (mant << 13);
    }
    float out;
    std::memcpy(&out, &f, 4);
    return out;
}

VNPU_API void VNPU_CALL vnpu_cluster_config_init(vnpu_cluster_config_t *config)
{
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->abi_version = VNPU_ABI_VERSION;
    config->num_streams = 1;
    config->request_timeout_ms = 30000;
    config->cluster_name = "vnpu-cluster";
}

VNPU_API void VNPU_CALL vnpu_speculative_config_init(vnpu_speculative_config_t *config)
{
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->abi_version = VNPU_ABI_VERSION;
    config->gamma = 4;
    config->vocab = 32000;
    config->max_tokens = 16;
    config->eos_token = 2;
    config->seed = 1;
}

VNPU_API void VNPU_CALL vnpu_node_config_init(vnpu_node_config_t *config)
{
    if (!config) return;
    std::memset(config, 0, sizeof(*config));
    config->abi_version = VNPU_ABI_VERSION;
    config->port = 9449;
    config->bind_address = "0.0.0.0";
    config->node_name = "vnpu-node";
}

// ---------------------------------------------------------------------------
// Device lifecycle (reference runtime.cpp:817-1152)
// ---------------------------------------------------------------------------

namespace {

enum : uint32_t { kTilesI8 = 1, kTilesF32 = 2 };

// Stores a tile triple (cull-mask sampling, device info) and derives the GEMM
// kernels it forces for the dtypes in `which`; the other dtype keeps its
// forced choice.  int8: the kernel named by gemm_i8_variant_for_tiles.  f32:
// 128 x depth x 128 fixes the K depth per workgroup of the split-K kernel.
void apply_tiles(vnpu_device_t *device, uint32_t tm, uint32_t tk, uint32_t tn, uint32_t which)
{
    device->tile_m.store(tm);
    device->tile_k.store(tk);
    device->tile_n.store(tn);
    device->info.tile_m = tm;
    device->info.tile_k = tk;
    device->info.tile_n = tn;
    if (which & kTilesI8) device->i8_variant.store(vnpu::k::gemm_i8_variant_for_tiles(tm, tk, tn));
    if (which & kTilesF32) device->f32_depth.store(tm == 128 && tn == 128 && tk % 16 == 0 ? tk : 0);
}

}  // namespace

VNPU_API vnpu_status_t VNPU_CALL vnpu_device_create(const vnpu_config_t *config,
                                                    vnpu_device_t **out_device)
{
    if (!out_device) return VNPU_ERR_INVALID_ARGUMENT;
    *out_device = nullptr;
    return guard([&]() -> vnpu_status_t {
        vnpu_config_t cfg;
        vnpu_config_init(&cfg);
        if (config) cfg = *config;
        if (cfg.abi_version == 0) cfg.abi_version = VNPU_ABI_VERSION;
        if (cfg.abi_version != VNPU_ABI_VERSION) return VNPU_ERR_UNSUPPORTED;

        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
            (void)hipGetLastError();
            debug_log("no HIP device visible: the MI355X backend needs a GPU");
            return VNPU_ERR_UNSUPPORTED;
        }
        int ordinal = 0;
        if (const char *e = std::getenv("VNPU_HIP_DEVICE")) ordinal = std::atoi(e);
        if (ordinal < 0 || ordinal >= count) return VNPU_ERR_INVALID_ARGUMENT;
        VNPU_HIP(hipSetDevice(ordinal));
        hipDeviceProp_t prop;
        VNPU_HIP(hipGetDeviceProperties(&prop, ordinal));

        // The allocation-free attention entry point's scratch address on
        // this device (the device is current).
        vnpu::k::attention_scratch_setup(ordinal);

        auto *d = new vnpu_device_t();
        d->config = cfg;
        d->hip_device = ordinal;
        d->cu_count = static_cast<uint32_t>(prop.multiProcessorCount);
        for (auto &r : d->regs) r.store(0);
        d->name = cfg.node_name ? cfg.node_name : "vnpu0";

        // The reference's AVX2 default tiles (runtime.cpp:923-933); on this
        // backend they only shape Wildcat cull-mask sampling.
        uint32_t tm = cfg.tile_m, tk = cfg.tile_k, tn = cfg.tile_n;
        if (!tm || !tk || !tn) {
            tm = 128;
            tk = 128;
            tn = 64;
        }
        apply_tiles(d, tm, tk, tn, kTilesI8 | kTilesF32);
        // ATTENTION_F32 rounds in the reference's order unless the caller
        // asks for throughput (VNPU_CONFIG_HIGH_THROUGHPUT, or
        // VNPU_REFERENCE_ORDER=0 for every device); VNPU_CONFIG_REFERENCE_ORDER
        // or VNPU_REFERENCE_ORDER=1 keep the reference's order regardless.
        // VNPU_WS_MAX_SPIN bounds the f32 GEMM's producer/consumer waits
        // (polls per wait): a test hook that forces the bounded-wait failure.
        if (const char *ms = std::getenv("VNPU_WS_MAX_SPIN"))
            d->ws_max_spin = static_cast<uint32_t>(std::strtoul(ms, nullptr, 10));
        const char *ro = std::getenv("VNPU_REFERENCE_ORDER");
        const bool fast = (cfg.flags & VNPU_CONFIG_HIGH_THROUGHPUT) != 0 || (ro && ro[0] == '0');
        d->reference_order = (cfg.flags & VNPU_CONFIG_REFERENCE_ORDER) != 0 || (ro && ro[0] == '1') || !fast;
        // "threads" = parallel units: the CU count unless the caller pins it.
        const uint32_t units = cfg.num_threads ? cfg.num_threads : d->cu_count;

        auto &info = d->info;
        std::memset(&info, 0, sizeof(info));
        info.abi_version = VNPU_ABI_VERSION;
        std::snprintf(info.name, sizeof(info.name), "%s", d->name.c_str());
        std::snprintf(info.vendor, sizeof(info.vendor), "AMD");
        std::snprintf(info.cpu_arch, sizeof(info.cpu_arch), "%s", prop.gcnArchName);
        std::snprintf(info.backend, sizeof(info.backend), "HIP %s (%s, %d CUs)", prop.gcnArchName,
                      prop.name, prop.multiProcessorCount);
        info.simd_bits = 64 * 32;  // one wave64 VGPR
        info.num_threads = units;
        info.num_compute_units = cfg.num_compute_units ? cfg.num_compute_units : d->cu_count;
        info.local_store_bytes = static_cast<uint32_t>(prop.maxSharedMemoryPerMultiProcessor
                                                           ? prop.maxSharedMemoryPerMultiProcessor
                                                           : prop.sharedMemPerBlock);
        info.tile_m = tm;
        info.tile_k = tk;
        info.tile_n = tn;
        info.physical_cores = d->cu_count;
        info.features = VNPU_FEATURE_THREADS | VNPU_FEATURE_TRACE | VNPU_FEATURE_GPU_FUTURE;
        info.l1d_bytes = 32 * 1024;
        info.l2_bytes = static_cast<uint64_t>(prop.l2CacheSize);
        info.l3_bytes = 256ull << 20;  // Infinity Cache
        info.total_memory_bytes = prop.totalGlobalMem;

        d->regs[VNPU_REG_ID / 4].store(VNPU_MAGIC);
        d->regs[VNPU_REG_VERSION / 4].store(VNPU_ABI_VERSION);
        d->regs[VNPU_REG_CONTROL / 4].store(1);
        d->regs[VNPU_REG_STATUS / 4].store(1);
        d->regs[VNPU_REG_ACTIVE_CUS / 4].store(info.num_compute_units);
        d->regs[VNPU_REG_CLOCK_MHZ / 4].store(static_cast<uint32_t>(prop.clockRate / 1000));
        d->regs[VNPU_REG_FEATURE_LO / 4].store(static_cast<uint32_t>(info.features & 0xffffffffu));
        d->regs[VNPU_REG_FEATURE_HI / 4].store(static_cast<uint32_t>(info.features >> 32));
        d->regs[VNPU_REG_IRQ_MASK / 4].store(0xffffffffu);
        d->trace.enabled.store((cfg.flags & VNPU_CONFIG_TRACE) != 0);
        d->trace.trace_file = cfg.trace_file ? cfg.trace_file : "";
        debug_log("created %s on HIP device %d (%s), %u CUs", d->name.c_str(), ordinal,
                  prop.gcnArchName, d->cu_count);
        *out_device = d;
        return VNPU_OK;
    });
}

static void destroy_stream_obj(vnpu_stream_t *s)
{
    if (!s) return;
    if (s->hip) {
        s->close_period();
        (void)hipStreamSynchronize(s->hip);
        s->resolve_timing(true);
        (void)hipStreamDestroy(s->hip);
    }
    for (hipEvent_t e : s->event_pool) (void)hipEventDestroy(e);
    if (s->workspace) (void)hipFree(s->workspace);
    if (s->staging) (void)hipFree(s->staging);
    if (s->cull_scratch) (void)hipFree(s->cull_scratch);
    if (s->err_host) (void)hipHostFree(s->err_host);
    delete s;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_trace_write_chrome(const vnpu_device_t *device,
                                                         const char *path);

VNPU_API void VNPU_CALL vnpu_device_destroy(vnpu_device_t *device)
{
    if (!device) return;
    std::vector<vnpu_stream_t *> streams;
    {
        std::lock_guard<std::mutex> lock(device->stream_mutex);
        streams.swap(device->streams);
    }
    (void)hipSetDevice(device->hip_device);
    for (auto *s : streams) destroy_stream_obj(s);
    if ((device->config.flags & VNPU_CONFIG_TRACE_CHROME) && !device->trace.trace_file.empty())
        vnpu_trace_write_chrome(device, device->trace.trace_file.c_str());
    device->trace.reset();
    release_device_tables(device);
    if (device->culled_dev) (void)hipFree(device->culled_dev);
    delete device;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_device_get_info(const vnpu_device_t *device,
                                                      vnpu_device_info_t *info)
{
    if (!device || !info) return VNPU_ERR_INVALID_ARGUMENT;
    *info = device->info;
    info->tile_m = device->tile_m.load();
    info->tile_k = device->tile_k.load();
    info->tile_n = device->tile_n.load();
    return VNPU_OK;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_device_get_status(const vnpu_device_t *device,
                                                        vnpu_device_status_t *status)
{
    if (!device || !status) return VNPU_ERR_INVALID_ARGUMENT;
    std::memset(status, 0, sizeof(*status));
    status->commands_submitted = device->commands_submitted.load();
    status->commands_completed = device->commands_completed.load();
    status->kernel_time_ns = device->kernel_ns.load();
    status->dispatch_time_ns = device->dispatch_ns.load();
    status->memory_time_ns = device->memory_ns.load();
    status->sync_time_ns = device->sync_ns.load();
    status->bytes_read = device->bytes_read.load();
    status->bytes_written = device->bytes_written.load();
    status->flops = device->flops.load();
    status->tiles_dispatched = device->tiles_dispatched.load();
    status->tiles_culled = device->tiles_culled.load();
    {
        // GPU-counted culls (device-resident masks): a copy only when any exist.
        auto *d = const_cast<vnpu_device_t *>(device);
        std::lock_guard<std::mutex> lock(d->culled_mutex);
        if (d->culled_dev) {
            unsigned long long v = 0;
            if (hipSetDevice(d->hip_device) == hipSuccess &&
                hipMemcpy(&v, d->culled_dev, sizeof(v), hipMemcpyDeviceToHost) == hipSuccess)
                status->tiles_culled += v;
            else
                (void)hipGetLastError();
        }
    }
    status->dma_bytes = device->dma_bytes.load();
    status->interrupts = device->interrupts.load();
    status->busy = device->busy.load();
    status->error = device->error.load();
    status->last_opcode = device->last_opcode.load();
    status->active_workers = device->active_workers.load();
    return VNPU_OK;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_device_reset(vnpu_device_t *device)
{
    if (!device) return VNPU_ERR_INVALID_ARGUMENT;
    if (device->busy.load()) return VNPU_ERR_DEVICE_BUSY;
    for (auto *a : {&device->commands_submitted, &device->commands_completed, &device->kernel_ns,
                    &device->dispatch_ns, &device->memory_ns, &device->sync_ns,
                    &device->bytes_read, &device->bytes_written, &device->flops,
                    &device->tiles_dispatched, &device->tiles_culled, &device->dma_bytes,
                    &device->interrupts})
        a->store(0);
    {
        std::lock_guard<std::mutex> lock(device->culled_mutex);
        if (device->culled_dev && (hipSetDevice(device->hip_device) != hipSuccess ||
                                   hipMemset(device->culled_dev, 0, sizeof(unsigned long long)) != hipSuccess))
            (void)hipGetLastError();
    }
    device->error.store(0);
    device->last_opcode.store(0);
    device->regs[VNPU_REG_ERROR / 4].store(0);
    device->regs[VNPU_REG_IRQ_STATUS / 4].store(0);
    device->trace.reset();
    return VNPU_OK;
}


VNPU_API vnpu_status_t VNPU_CALL vnpu_device_set_tiles(vnpu_device_t *device, uint32_t tile_m,
                                                       uint32_t tile_k, uint32_t tile_n)
{
    if (!device || !tile_m || !tile_k || !tile_n) return VNPU_ERR_INVALID_ARGUMENT;
    apply_tiles(device, tile_m, tile_k, tile_n, kTilesI8 | kTilesF32);
    return VNPU_OK;
}

// MMIO register file (reference runtime.cpp:1102-1138)
VNPU_API uint32_t VNPU_CALL vnpu_mmio_read32(vnpu_device_t *device, uint32_t offset)
{
    if (!device || (offset & 3u)) return 0xffffffffu;
    const uint32_t idx = offset / 4;
    if (idx >= VNPU_REG_COUNT) return 0xffffffffu;
    switch (offset) {
    case VNPU_REG_STATUS: return 1u | (device->busy.load() ? 2u : 0u);
    case VNPU_REG_ERROR: return device->regs[idx].load() | (device->error.load() ? 1u : 0u);
    case VNPU_REG_CMD_HEAD: return static_cast<uint32_t>(device->commands_completed.load());
    case VNPU_REG_CMD_TAIL: return static_cast<uint32_t>(device->commands_submitted.load());
    case VNPU_REG_ACTIVE_CUS: return device->active_workers.load();
    case VNPU_REG_THERMAL: return 0;
    default: return device->regs[idx].load();
    }
}

VNPU_API void VNPU_CALL vnpu_mmio_write32(vnpu_device_t *device, uint32_t offset, uint32_t value)
{
    if (!device || (offset & 3u)) return;
    const uint32_t idx = offset / 4;
    if (idx >= VNPU_REG_COUNT) return;
    device->regs[idx].store(value);
    if (offset == VNPU_REG_DOORBELL && value)
        device->raise_irq(1u << 0);
    else if (offset == VNPU_REG_CONTROL && (value & 2u))
        vnpu_device_reset(device);
    else if (offset == VNPU_REG_IRQ_STATUS)
        device->regs[idx].store(0);
}

VNPU_API void VNPU_CALL vnpu_device_set_interrupt_callback(vnpu_device_t *device,
                                                           vnpu_interrupt_cb_t cb, void *user_data)
{
    if (!device) return;
    std::lock_guard<std::mutex> lock(device->irq_mutex);
    device->irq_cb = cb;
    device->irq_user = user_data;
}

// ---------------------------------------------------------------------------
// Events (reference runtime.cpp:1154-1209)
// ---------------------------------------------------------------------------

VNPU_API vnpu_status_t VNPU_CALL vnpu_event_create(vnpu_event_t **out_event)
{
    if (!out_event) return VNPU_ERR_INVALID_ARGUMENT;
    *out_event = nullptr;
    return guard([&]() -> vnpu_status_t {
        *out_event = new vnpu_event_t();
        return VNPU_OK;
    });
}

VNPU_API void VNPU_CALL vnpu_event_destroy(vnpu_event_t *event)
{
    if (!event) return;
    if (event->hip) {
        (void)hipSetDevice(event->hip_device);
        (void)hipEventSynchronize(event->hip);
        (void)hipEventDestroy(event->hip);
    }
    delete event;
}

// Signalled = a batch was submitted with this event and the GPU passed it.
static int event_ready(vnpu_event_t *e)
{
    if (e->host_signaled) return 1;
    if (!e->submitted || !e->hip) return 0;
    const hipError_t q = hipEventQuery(e->hip);
    if (q == hipSuccess) return 1;
    if (q == hipErrorNotReady) return 0;
    (void)hipGetLastError();
    return -1;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_event_wait(vnpu_event_t *event, uint32_t timeout_ms)
{
    if (!event) return VNPU_ERR_INVALID_ARGUMENT;
    const auto deadline = std::chrono::steady_clock::now() + std::chrono::milliseconds(timeout_ms);
    for (;;) {
        {
            std::lock_guard<std::mutex> lock(event->mutex);
            const int r = event_ready(event);
            if (r > 0) return event->status;
            if (r < 0) return VNPU_ERR_DEVICE_ERROR;
        }
        if (std::chrono::steady_clock::now() >= deadline) return VNPU_ERR_TIMEOUT;
        std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_event_query(const vnpu_event_t *event)
{
    if (!event) return VNPU_ERR_INVALID_ARGUMENT;
    auto *e = const_cast<vnpu_event_t *>(event);
    std::lock_guard<std::mutex> lock(e->mutex);
    return event_ready(e) > 0 ? VNPU_OK : VNPU_ERR_DEVICE_BUSY;
}

// ---------------------------------------------------------------------------
// Streams (reference runtime.cpp:1215-1361)
// ---------------------------------------------------------------------------

VNPU_API vnpu_status_t VNPU_CALL vnpu_stream_create(vnpu_device_t *device, int priority,
                                                    vnpu_stream_t **out_stream)
{
    if (!device || !out_stream) return VNPU_ERR_INVALID_ARGUMENT;
    *out_stream = nullptr;
    return guard([&]() -> vnpu_status_t {
        VNPU_HIP(hipSetDevice(device->hip_device));
        auto *s = new vnpu_stream_t();
        s->device = device;
        s->priority = priority;  // recorded only: every stream runs at default priority
        hipError_t e = hipStreamCreate(&s->hip);
        if (e == hipSuccess)
            e = hipHostMalloc(reinterpret_cast<void **>(&s->err_host), sizeof(uint32_t),
                              hipHostMallocMapped | hipHostMallocCoherent);
        if (e == hipSuccess) {
            *s->err_host = 0;
            e = hipHostGetDevicePointer(reinterpret_cast<void **>(&s->err_dev), s->err_host, 0);
        }
        if (e != hipSuccess) {
            (void)hipGetLastError();
            destroy_stream_obj(s);
            return VNPU_ERR_DEVICE_ERROR;
        }
        {
            std::lock_guard<std::mutex> lock(device->stream_mutex);
            device->streams.push_back(s);
        }
        *out_stream = s;
        return VNPU_OK;
    });
}

VNPU_API void VNPU_CALL vnpu_stream_destroy(vnpu_stream_t *stream)
{
    if (!stream) return;
    if (vnpu_device_t *d = stream->device) {
        std::lock_guard<std::mutex> lock(d->stream_mutex);
        auto &v = d->streams;
        v.erase(std::remove(v.begin(), v.end(), stream), v.end());
        (void)hipSetDevice(d->hip_device);
    }
    destroy_stream_obj(stream);
}

VNPU_API void *VNPU_CALL vnpu_stream_hip_handle(vnpu_stream_t *stream)
{
    return stream ? static_cast<void *>(stream->hip) : nullptr;
}

// ATTENTION_F32 that allocates nothing (no reference counterpart): for
// callers that cannot allocate device memory, such as code under HIP graph
// capture or a serving loop.  The kernels are vnpu_attention_f32's; their
// scratch is the per-GPU device array of attention.hip (set up by
// vnpu_device_create), shared by every call on that GPU, so calls that
// overlap on one GPU (two streams, two threads) race.  Enqueues only.
VNPU_API vnpu_status_t VNPU_CALL vnpu_attention_f32_noalloc(vnpu_stream_t *stream,
                                                            const vnpu_attention_f32_args_t *args)
{
    if (!stream || !args) return VNPU_ERR_INVALID_ARGUMENT;
    vnpu_device_t *d = stream->device;
    try {
        ExecStats st;
        std::lock_guard<std::mutex> lock(stream->mutex);
        VNPU_HIP(hipSetDevice(d->hip_device));
        enqueue_attention_noalloc(stream, *args, st);
        d->bytes_read.fetch_add(st.bytes_read);
        d->bytes_written.fetch_add(st.bytes_written);
        d->flops.fetch_add(st.flops);
        d->last_opcode.store(VNPU_OP_ATTENTION_F32);
        return VNPU_OK;
    } catch (const ArgError &e) {
        debug_log("vnpu_attention_f32_noalloc: %s", e.what());
        return VNPU_ERR_INVALID_ARGUMENT;
    } catch (const std::exception &e) {
        // A launch failure: the stream's error becomes sticky, as for a
        // failed command of a batch.
        debug_log("vnpu_attention_f32_noalloc: %s", e.what());
        (void)hipGetLastError();
        const uint32_t code = static_cast<uint32_t>(-VNPU_ERR_INTERNAL);
        d->error.store(code);
        d->regs[VNPU_REG_ERROR / 4].store(code);
        stream->last_error.store(code);
        return VNPU_ERR_INTERNAL;
    } catch (...) {
        return VNPU_ERR_INTERNAL;
    }
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_stream_sync(vnpu_stream_t *stream)
{
    if (!stream) return VNPU_ERR_INVALID_ARGUMENT;
    const uint64_t t0 = now_ns();
    hipError_t e;
    {
        std::lock_guard<std::mutex> lock(stream->mutex);
        (void)hipSetDevice(stream->device->hip_device);
        stream->close_period();
        e = hipStreamSynchronize(stream->hip);
        if (e == hipSuccess) stream->resolve_timing(true);
    }
    vnpu_device_t *d = stream->device;
    d->sync_ns.fetch_add(now_ns() - t0);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        const uint32_t code = static_cast<uint32_t>(-VNPU_ERR_DEVICE_ERROR);
        stream->last_error.store(code);
        d->error.store(code);
        d->regs[VNPU_REG_ERROR / 4].store(code);
    } else if (stream->err_host && __atomic_exchange_n(stream->err_host, 0u, __ATOMIC_ACQ_REL) != 0) {
        // A kernel's bounded wait gave up (its output is not valid): a
        // failed command, sticky on this stream as in the reference
        // (runtime.cpp:1248-1254, 1281-1289).
        debug_log("vnpu_stream_sync: a kernel's bounded wait gave up; its output is invalid");
        const uint32_t code = static_cast<uint32_t>(-VNPU_ERR_INTERNAL);
        stream->last_error.store(code);
        d->error.store(code);
        d->regs[VNPU_REG_ERROR / 4].store(code);
    }
    const uint64_t pend = stream->pending.exchange(0);
    d->commands_completed.fetch_add(pend);
    d->regs[VNPU_REG_CMD_HEAD / 4].store(static_cast<uint32_t>(d->commands_completed.load()));
    return stream->last_error.load() ? VNPU_ERR_DEVICE_ERROR : VNPU_OK;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_stream_submit(vnpu_stream_t *stream,
                                                    const vnpu_command_t *commands, uint64_t count,
                                                    vnpu_event_t *event)
{
    if (!stream || (!commands && count) || count > (1u << 24)) return VNPU_ERR_INVALID_ARGUMENT;
    if (count == 0) {
        if (event) {
            std::lock_guard<std::mutex> lock(event->mutex);
            event->host_signaled = true;
            event->status = VNPU_OK;
        }
        return VNPU_OK;
    }
    return guard([&]() -> vnpu_status_t {
        vnpu_device_t *d = stream->device;
        uint32_t flags = 0;
        for (uint64_t i = 0; i < count; ++i) flags |= commands[i].flags;
        d->commands_submitted.fetch_add(count);
        d->regs[VNPU_REG_CMD_TAIL / 4].store(static_cast<uint32_t>(d->commands_submitted.load()));
        stream->pending.fetch_add(count);
        vnpu_status_t batch_status = VNPU_OK;
        const bool tracing = d->trace.enabled.load();
        std::lock_guard<std::mutex> lock(stream->mutex);
        VNPU_HIP(hipSetDevice(d->hip_device));
        d->busy.fetch_add(1);
        d->active_workers.fetch_add(1);
        if (stream->batch_timing.size() >= 256) stream->resolve_timing(false);
        stream->open_period();
        auto account = [&](const ExecStats &st, uint64_t host) {
            d->dispatch_ns.fetch_add(host);
            d->bytes_read.fetch_add(st.bytes_read);
            d->bytes_written.fetch_add(st.bytes_written);
            d->flops.fetch_add(st.flops);
            d->dma_bytes.fetch_add(st.dma_bytes);
            d->tiles_dispatched.fetch_add(st.tiles_dispatched);
            d->tiles_culled.fetch_add(st.tiles_culled);
        };
        // A failed command marks the batch, the device error register and the
        // stream's sticky error.
        auto fail = [&](vnpu_status_t rc) {
            batch_status = rc;
            const uint32_t code = static_cast<uint32_t>(-rc);
            d->error.store(code);
            d->regs[VNPU_REG_ERROR / 4].store(code);
            stream->last_error.store(code);
        };
        for (uint64_t i = 0; i < count; ++i) {
            const vnpu_command_t &cmd = commands[i];
            const uint64_t t0 = now_ns();
            // Two independent MATMUL_I8 in a row may share one launch (not
            // while tracing, which times every command on the GPU).
            if (!tracing && i + 1 < count && cmd.opcode == VNPU_OP_MATMUL_I8 &&
                commands[i + 1].opcode == VNPU_OP_MATMUL_I8) {
                ExecStats s0, s1;
                bool paired = false;
                try {
                    paired = try_execute_pair(d, stream, cmd, commands[i + 1], flags, s0, s1);
                } catch (const std::exception &ex) {
                    debug_log("paired matmul_i8 failed: %s", ex.what());
                    (void)hipGetLastError();
                    fail(VNPU_ERR_INTERNAL);
                    ++i;
                    continue;
                }
                if (paired) {
                    d->last_opcode.store(VNPU_OP_MATMUL_I8);
                    const uint64_t host = now_ns() - t0;
                    account(s0, host / 2);
                    account(s1, host - host / 2);
                    ++i;
                    continue;
                }
            }
            // A decode-sized MATMUL_I8 and an ADD of its output may share the
            // GEMV's launch (not while tracing).
            if (!tracing && i + 1 < count && cmd.opcode == VNPU_OP_MATMUL_I8 &&
                commands[i + 1].opcode == VNPU_OP_ADD_F32) {
                ExecStats s0, s1;
                bool fused = false;
                try {
                    fused = try_execute_matmul_add(d, stream, cmd, commands[i + 1], flags, s0, s1);
                } catch (const std::exception &ex) {
                    debug_log("matmul_i8 + add failed: %s", ex.what());
                    (void)hipGetLastError();
                    fail(VNPU_ERR_INTERNAL);
                    ++i;
                    continue;
                }
                if (fused) {
                    d->last_opcode.store(VNPU_OP_ADD_F32);
                    const uint64_t host = now_ns() - t0;
                    account(s0, host / 2);
                    account(s1, host - host / 2);
                    ++i;
                    continue;
                }
            }
            // ADD / SWIGLU / RMSNORM followed by the row commands that consume
            // their output may run as one row-chain kernel (not while tracing).
            if (!tracing && i + 1 < count &&
                (cmd.opcode == VNPU_OP_ADD_F32 || cmd.opcode == VNPU_OP_SWIGLU_F32 ||
                 cmd.opcode == VNPU_OP_RMSNORM_F32)) {
                ExecStats cs[3];
                uint32_t matched = 0, used = 0;
                try {
                    used = try_execute_chain(stream, commands + i, count - i, &matched, cs);
                } catch (const std::exception &ex) {
                    debug_log("row chain failed: %s", ex.what());
                    (void)hipGetLastError();
                    fail(VNPU_ERR_INTERNAL);
                    i += matched ? matched - 1 : 0;
                    continue;
                }
                if (used) {
                    d->last_opcode.store(commands[i + used - 1].opcode);
                    const uint64_t host = now_ns() - t0;
                    const uint64_t share = host / used;
                    for (uint32_t k = 0; k < used; ++k) account(cs[k], k + 1 < used ? share : host - share * (used - 1));
                    i += used - 1;
                    continue;
                }
            }
            TraceRecord rec;
            if (tracing) {
                {
                    std::lock_guard<std::mutex> tl(d->trace.mutex);
                    if (!d->trace.epoch && create_timing_event(&d->trace.epoch) == hipSuccess)
                        (void)hipEventRecord(d->trace.epoch, stream->hip);
                }
                if (create_timing_event(&rec.start) == hipSuccess) (void)hipEventRecord(rec.start, stream->hip);
            }
            ExecStats st;
            vnpu_status_t rc = VNPU_OK;
            if (cmd.opcode >= VNPU_OP_COUNT) {
                rc = VNPU_ERR_INVALID_COMMAND;
            } else {
                try {
                    d->last_opcode.store(cmd.opcode);
                    execute_command(d, stream, cmd, flags, st);
                } catch (const std::exception &ex) {
                    debug_log("command %s failed: %s", vnpu_opcode_name(cmd.opcode), ex.what());
                    (void)hipGetLastError();
                    rc = VNPU_ERR_INTERNAL;
                }
            }
            const uint64_t host = now_ns() - t0;
            const uint32_t cat = trace_category(cmd.opcode);
            if (cat == 1) d->memory_ns.fetch_add(host);
            if (cat == 2) d->sync_ns.fetch_add(host);
            account(st, host);
            if (tracing) {
                if (create_timing_event(&rec.stop) == hipSuccess) (void)hipEventRecord(rec.stop, stream->hip);
                rec.opcode = cmd.opcode;
                rec.unit = st.unit;
                rec.id = cmd.id;
                rec.bytes_read = st.bytes_read;
                rec.bytes_written = st.bytes_written;
                rec.flops = st.flops;
                rec.host_ns = host;
                if (rc != VNPU_OK) {
                    if (rec.start) (void)hipEventDestroy(rec.start);
                    if (rec.stop) (void)hipEventDestroy(rec.stop);
                } else {
                    std::lock_guard<std::mutex> tl(d->trace.mutex);
                    if (d->trace.records.size() < 200000) d->trace.records.push_back(rec);
                    else {
                        (void)hipEventDestroy(rec.start);
                        (void)hipEventDestroy(rec.stop);
                    }
                }
            }
            if (rc != VNPU_OK) fail(rc);
        }
        if (++stream->period_batches >= 256) stream->close_period();
        if (event) {
            std::lock_guard<std::mutex> el(event->mutex);
            if (event->hip && event->hip_device != d->hip_device) {
                (void)hipEventDestroy(event->hip);
                event->hip = nullptr;
            }
            if (!event->hip) {
                VNPU_HIP(hipEventCreateWithFlags(&event->hip, hipEventDisableTiming));
                event->hip_device = d->hip_device;
            }
            VNPU_HIP(hipEventRecord(event->hip, stream->hip));
            event->submitted = true;
            event->host_signaled = false;
            event->status = batch_status;
            event->command_count = count;
        }
        d->active_workers.fetch_sub(1);
        d->busy.fetch_sub(1);
        d->raise_irq(1u << 1);
        return VNPU_OK;
    });
}

// ---------------------------------------------------------------------------
// Buffers (reference runtime.cpp:1367-1440): HBM allocations.
// ---------------------------------------------------------------------------

VNPU_API vnpu_status_t VNPU_CALL vnpu_buffer_alloc(vnpu_device_t *device, uint64_t bytes,
                                                   vnpu_buffer_t **out_buffer)
{
    if (!device || !bytes || !out_buffer) return VNPU_ERR_INVALID_ARGUMENT;
    *out_buffer = nullptr;
    return guard([&]() -> vnpu_status_t {
        VNPU_HIP(hipSetDevice(device->hip_device));
        void *p = nullptr;
        if (hipMalloc(&p, static_cast<size_t>(bytes)) != hipSuccess) {
            (void)hipGetLastError();
            return VNPU_ERR_OUT_OF_MEMORY;
        }
        if (hipMemset(p, 0, static_cast<size_t>(bytes)) != hipSuccess) {
            (void)hipFree(p);
            return VNPU_ERR_DEVICE_ERROR;
        }
        auto *b = new vnpu_buffer_t();
        register_device_range(p, static_cast<size_t>(bytes));
        b->device = device;
        b->dev_ptr = p;
        b->bytes = bytes;
        static std::atomic<uint64_t> next{1};
        b->handle = next.fetch_add(1);
        *out_buffer = b;
        return VNPU_OK;
    });
}

VNPU_API void VNPU_CALL vnpu_buffer_free(vnpu_buffer_t *buffer)
{
    if (!buffer) return;
    if (buffer->dev_ptr) {
        unregister_device_range(buffer->dev_ptr);
        (void)hipSetDevice(buffer->device->hip_device);
        (void)hipFree(buffer->dev_ptr);
    }
    delete buffer;
}

VNPU_API void *VNPU_CALL vnpu_buffer_host_ptr(vnpu_buffer_t *buffer)
{
    return buffer ? buffer->dev_ptr : nullptr;
}

VNPU_API uint64_t VNPU_CALL vnpu_buffer_size(const vnpu_buffer_t *buffer)
{
    return buffer ? buffer->bytes : 0;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_buffer_copy(vnpu_stream_t *stream, void *dst, const void *src,
                                                  uint64_t bytes, uint32_t direction)
{
    if (!stream || !dst || !src || !bytes) return VNPU_ERR_INVALID_ARGUMENT;
    vnpu_command_t cmd{};
    cmd.opcode = VNPU_OP_COPY;
    cmd.args.copy.dst = dst;
    cmd.args.copy.src = src;
    cmd.args.copy.bytes = bytes;
    cmd.args.copy.direction = direction;
    vnpu_status_t rc = vnpu_stream_submit(stream, &cmd, 1, nullptr);
    if (rc != VNPU_OK) return rc;
    return vnpu_stream_sync(stream);
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_buffer_memset(vnpu_stream_t *stream, void *dst, uint32_t value,
                                                    uint64_t bytes)
{
    if (!stream || !dst || !bytes) return VNPU_ERR_INVALID_ARGUMENT;
    vnpu_command_t cmd{};
    cmd.opcode = VNPU_OP_MEMSET;
    cmd.args.memset.dst = dst;
    cmd.args.memset.value = value;
    cmd.args.memset.bytes = bytes;
    vnpu_status_t rc = vnpu_stream_submit(stream, &cmd, 1, nullptr);
    if (rc != VNPU_OK) return rc;
    return vnpu_stream_sync(stream);
}

// ---------------------------------------------------------------------------
// Packed weights
// ---------------------------------------------------------------------------

VNPU_API vnpu_status_t VNPU_CALL vnpu_pack_weights_i8(vnpu_device_t *device, const int8_t *B,
                                                      const float *scales, uint32_t K, uint32_t N,
                                                      uint32_t ldb, uint32_t trans_b,
                                                      vnpu_packed_weights_t **out_weights)
{
    if (!device || !B || !out_weights || !K || !N || trans_b > 1) return VNPU_ERR_INVALID_ARGUMENT;
    *out_weights = nullptr;
    const uint32_t ld = ldb ? ldb : (trans_b ? K : N);
    if (ld < (trans_b ? K : N)) return VNPU_ERR_INVALID_ARGUMENT;
    return guard([&]() -> vnpu_status_t {
        *out_weights = pack_weights(device, B, scales, K, N, ldb, trans_b);
        return VNPU_OK;
    });
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_pack_weights_i8_masked(vnpu_device_t *device, const int8_t *B,
                                                             const float *scales, uint32_t K, uint32_t N,
                                                             uint32_t ldb, uint32_t trans_b,
                                                             const uint8_t *tile_mask, uint32_t mask_ld,
                                                             vnpu_packed_weights_t **out_weights)
{
    if (!device || !B || !out_weights || !K || !N || trans_b > 1) return VNPU_ERR_INVALID_ARGUMENT;
    *out_weights = nullptr;
    const uint32_t ld = ldb ? ldb : (trans_b ? K : N);
    if (ld < (trans_b ? K : N)) return VNPU_ERR_INVALID_ARGUMENT;
    if (tile_mask && mask_ld && mask_ld < (N + 63) / 64) return VNPU_ERR_INVALID_ARGUMENT;
    return guard([&]() -> vnpu_status_t {
        *out_weights = pack_weights(device, B, scales, K, N, ldb, trans_b, tile_mask, mask_ld);
        return VNPU_OK;
    });
}

VNPU_API void VNPU_CALL vnpu_packed_weights_destroy(vnpu_packed_weights_t *weights)
{
    destroy_packed(weights);
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_packed_weights_info(const vnpu_packed_weights_t *weights,
                                                          uint32_t *K, uint32_t *N, uint64_t *bytes,
                                                          const float **scales,
                                                          const int32_t **column_sums)
{
    if (!weights) return VNPU_ERR_INVALID_ARGUMENT;
    if (K) *K = weights->K;
    if (N) *N = weights->N;
    if (bytes) *bytes = weights->frag_bytes;
    if (scales) *scales = weights->scales.data();
    if (column_sums) *column_sums = weights->column_sums.data();
    return VNPU_OK;
}

// ---------------------------------------------------------------------------
// Synchronous wrappers (reference scheduler.cpp:864-902)
// ---------------------------------------------------------------------------

#define VNPU_SYNC_WRAPPER(fn, op, field, type)                                \
    VNPU_API vnpu_status_t VNPU_CALL fn(vnpu_stream_t *stream, const type *args) \
    {                                                                          \
        if (!stream || !args) return VNPU_ERR_INVALID_ARGUMENT;                \
        vnpu_command_t cmd{};                                                  \
        cmd.opcode = op;                                                       \
        cmd.args.field = *args;                                                \
        vnpu_status_t rc = vnpu_stream_submit(stream, &cmd, 1, nullptr);       \
        if (rc != VNPU_OK) return rc;                                          \
        return vnpu_stream_sync(stream);                                       \
    }

VNPU_SYNC_WRAPPER(vnpu_matmul_f32, VNPU_OP_MATMUL_F32, matmul_f32, vnpu_matmul_f32_args_t)
VNPU_SYNC_WRAPPER(vnpu_matmul_i8, VNPU_OP_MATMUL_I8, matmul_i8, vnpu_matmul_i8_args_t)
VNPU_SYNC_WRAPPER(vnpu_quantize_i8, VNPU_OP_QUANTIZE_I8, quantize_i8, vnpu_quantize_i8_args_t)
VNPU_SYNC_WRAPPER(vnpu_rmsnorm_f32, VNPU_OP_RMSNORM_F32, rmsnorm, vnpu_rmsnorm_f32_args_t)
VNPU_SYNC_WRAPPER(vnpu_softmax_f32, VNPU_OP_SOFTMAX_F32, softmax, vnpu_softmax_f32_args_t)
VNPU_SYNC_WRAPPER(vnpu_rope_f32, VNPU_OP_ROPE_F32, rope, vnpu_rope_f32_args_t)
VNPU_SYNC_WRAPPER(vnpu_swiglu_f32, VNPU_OP_SWIGLU_F32, swiglu, vnpu_swiglu_f32_args_t)
VNPU_SYNC_WRAPPER(vnpu_gelu_f32, VNPU_OP_GELU_F32, unary, vnpu_unary_f32_args_t)
VNPU_SYNC_WRAPPER(vnpu_add_f32, VNPU_OP_ADD_F32, binary, vnpu_binary_f32_args_t)
VNPU_SYNC_WRAPPER(vnpu_mul_f32, VNPU_OP_MUL_F32, binary, vnpu_binary_f32_args_t)
VNPU_SYNC_WRAPPER(vnpu_attention_f32, VNPU_OP_ATTENTION_F32, attention, vnpu_attention_f32_args_t)
VNPU_SYNC_WRAPPER(vnpu_mtp_head_f32, VNPU_OP_MTP_HEAD_F32, mtp_head, vnpu_mtp_head_f32_args_t)

#undef VNPU_SYNC_WRAPPER

// ---------------------------------------------------------------------------
// Sherlock trace (reference runtime.cpp:327-627, 1442-1479) on hipEvents.
// ---------------------------------------------------------------------------

VNPU_API vnpu_status_t VNPU_CALL vnpu_trace_enable(vnpu_device_t *device, int enable)
{
    if (!device) return VNPU_ERR_INVALID_ARGUMENT;
    device->trace.enabled.store(enable != 0);
    if (enable) device->trace.reset();
    return VNPU_OK;
}

VNPU_API void VNPU_CALL vnpu_trace_reset(vnpu_device_t *device)
{
    if (device) device->trace.reset();
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_trace_get_summary(const vnpu_device_t *device,
                                                        vnpu_trace_summary_t *summary)
{
    if (!device || !summary) return VNPU_ERR_INVALID_ARGUMENT;
    auto &tr = const_cast<vnpu_device_t *>(device)->trace;
    tr.resolve();
    std::memset(summary, 0, sizeof(*summary));
    std::lock_guard<std::mutex> lock(tr.mutex);
    uint64_t per_op[VNPU_OP_COUNT] = {};
    for (const auto &r : tr.records) {
        summary->events++;
        summary->total_time_ns += r.gpu_ns;
        const uint32_t cat = trace_category(r.opcode);
        if (cat == 0) summary->compute_time_ns += r.gpu_ns;
        else if (cat == 1) summary->memory_time_ns += r.gpu_ns;
        else summary->sync_time_ns += r.gpu_ns;
        summary->dispatch_time_ns += r.host_ns > r.gpu_ns ? r.host_ns - r.gpu_ns : 0;
        summary->bytes_read += r.bytes_read;
        summary->bytes_written += r.bytes_written;
        summary->flops += r.flops;
        if (r.opcode < VNPU_OP_COUNT) per_op[r.opcode] += r.gpu_ns;
    }
    if (summary->total_time_ns) {
        const double s = static_cast<double>(summary->total_time_ns) * 1e-9;
        summary->achieved_gflops = static_cast<double>(summary->flops) / s * 1e-9;
        summary->achieved_gbytes_s =
            static_cast<double>(summary->bytes_read + summary->bytes_written) / s * 1e-9;
    }
    for (uint32_t op = 0; op < VNPU_OP_COUNT; ++op)
        if (per_op[op] > summary->hot_time_ns) {
            summary->hot_time_ns = per_op[op];
            summary->hot_opcode = op;
        }
    summary->trace_overhead_ns = 0.0;
    return VNPU_OK;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_trace_dump(const vnpu_device_t *device, const char *path)
{
    if (!device) return VNPU_ERR_INVALID_ARGUMENT;
    vnpu_trace_summary_t s;
    vnpu_trace_get_summary(device, &s);
    std::ostringstream o;
    o << "vnpu trace (" << device->info.backend << ")\n"
      << "events " << s.events << ", gpu time " << s.total_time_ns / 1e6 << " ms\n"
      << "compute " << s.compute_time_ns / 1e6 << " ms, memory " << s.memory_time_ns / 1e6
      << " ms, sync " << s.sync_time_ns / 1e6 << " ms, host dispatch " << s.dispatch_time_ns / 1e6
      << " ms\n"
      << "achieved " << s.achieved_gflops << " GFLOP/s, " << s.achieved_gbytes_s << " GB/s\n"
      << "hot opcode " << vnpu_opcode_name(s.hot_opcode) << " (" << s.hot_time_ns / 1e6 << " ms)\n";
    const std::string text = o.str();
    if (!path || !*path) {
        std::fputs(text.c_str(), stderr);
        return VNPU_OK;
    }
    std::ofstream f(path);
    if (!f) return VNPU_ERR_IO;
    f << text;
    return f ? VNPU_OK : VNPU_ERR_IO;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_trace_write_chrome(const vnpu_device_t *device, const char *path)
{
    // The reference's Chrome trace layout (src/core/runtime.cpp:530-580):
    // complete events named OPCODE#id with a category, timestamps relative to
    // the first event at 1 ns resolution, args {op, unit, bytes_read,
    // bytes_written, flops}.  Start times and durations here are the GPU's
    // (hipEvent pairs around each command on its stream).
    if (!device || !path) return VNPU_ERR_INVALID_ARGUMENT;
    auto &tr = const_cast<vnpu_device_t *>(device)->trace;
    tr.resolve();
    std::ofstream f(path);
    if (!f) return VNPU_ERR_IO;
    std::lock_guard<std::mutex> lock(tr.mutex);
    uint64_t t0 = tr.records.empty() ? 0u : tr.records[0].gpu_start_ns;
    for (const auto &r : tr.records) t0 = std::min(t0, r.gpu_start_ns);
    static const char *cats[] = {"compute", "memory", "sync"};
    f << "{\n\"traceEvents\":[\n";
    f << "{\"name\":\"process_name\",\"ph\":\"M\",\"pid\":1,\"tid\":0,\"args\":{\"name\":\"VNPU "
      << device->info.name << "\"}}" << (tr.records.empty() ? "" : ",") << "\n";
    for (size_t i = 0; i < tr.records.size(); ++i) {
        const auto &r = tr.records[i];
        char buf[512];
        std::snprintf(buf, sizeof(buf),
                      "{\"name\":\"%s#%llu\",\"cat\":\"%s\",\"ph\":\"X\",\"ts\":%.3f,\"dur\":%.3f,"
                      "\"pid\":1,\"tid\":0,\"args\":{\"op\":\"%s\",\"unit\":\"%s\",\"bytes_read\":%llu,"
                      "\"bytes_written\":%llu,\"flops\":%llu}}%s\n",
                      vnpu_opcode_name(r.opcode), static_cast<unsigned long long>(r.id),
                      cats[trace_category(r.opcode)], static_cast<double>(r.gpu_start_ns - t0) / 1000.0,
                      static_cast<double>(r.gpu_ns) / 1000.0, vnpu_opcode_name(r.opcode),
                      vnpu_unit_name(r.unit), static_cast<unsigned long long>(r.bytes_read),
                      static_cast<unsigned long long>(r.bytes_written),
                      static_cast<unsigned long long>(r.flops), i + 1 < tr.records.size() ? "," : "");
        f << buf;
    }
    f << "],\n\"displayTimeUnit\":\"ns\",\"otherData\":{\"version\":\"" << vnpu_version_string()
      << "\"}}\n";
    return f ? VNPU_OK : VNPU_ERR_IO;
}

// ---------------------------------------------------------------------------
// Autotune (reference autotune.cpp:153-281): the candidates are this
// backend's GEMM kernels, named by tile triples that vnpu_device_set_tiles
// understands (int8: 256x128x256 wide, 256x128x128 8-wave, 256x64x128 64-deep,
// 128x64x128 generic; f32: 128 x depth x 128 with the K depth per workgroup).
// Each candidate the shape admits is timed on the GPU (hipEvents, best of
// `iterations`), the baseline is the automatic choice with the tiles the
// device had, and the fastest is written back with vnpu_device_set_tiles.
// As in the reference, tracing is off while tuning, iterations are clamped
// to 1..20 (0 means 3) and bytes_read counts 4-byte elements.
// ---------------------------------------------------------------------------

VNPU_API vnpu_status_t VNPU_CALL vnpu_autotune_gemm(vnpu_device_t *device, uint32_t M, uint32_t K,
                                                    uint32_t N, uint32_t iterations,
                                                    vnpu_dtype_t dtype, vnpu_tune_result_t *result)
{
    if (!device || !result || !M || !K || !N) return VNPU_ERR_INVALID_ARGUMENT;
    if (dtype != VNPU_DTYPE_F32 && dtype != VNPU_DTYPE_I8) return VNPU_ERR_UNSUPPORTED;
    if (iterations == 0) iterations = 3;
    if (iterations > 20) iterations = 20;
    return guard([&]() -> vnpu_status_t {
        std::memset(result, 0, sizeof(*result));
        const uint32_t orig_tm = device->tile_m.load(), orig_tk = device->tile_k.load(),
                       orig_tn = device->tile_n.load();
        // Only the tuned dtype's forced kernel changes; the other dtype's
        // choice is left as it was.
        const uint32_t which = dtype == VNPU_DTYPE_I8 ? kTilesI8 : kTilesF32;
        const uint32_t orig_i8 = device->i8_variant.load(), orig_f32 = device->f32_depth.load();
        auto restore_tiles = [&]() {
            apply_tiles(device, orig_tm, orig_tk, orig_tn, 0);
            device->i8_variant.store(orig_i8);
            device->f32_depth.store(orig_f32);
        };
        const bool trace_was_on = device->trace.enabled.exchange(false);
        struct Restore {
            vnpu_device_t *d;
            bool trace;
            ~Restore() { d->trace.enabled.store(trace); }
        } restore{device, trace_was_on};
        vnpu_stream_t *s = nullptr;
        vnpu_status_t rc = vnpu_stream_create(device, 0, &s);
        if (rc != VNPU_OK) return rc;
        struct StreamGuard {
            vnpu_stream_t *s;
            ~StreamGuard() { vnpu_stream_destroy(s); }
        } sgd{s};
        const bool i8 = dtype == VNPU_DTYPE_I8;
        const size_t ea = i8 ? 1 : 4;
        void *A = nullptr, *B = nullptr, *C = nullptr;
        VNPU_HIP(hipMalloc(&A, static_cast<size_t>(M) * K * ea));
        VNPU_HIP(hipMalloc(&B, static_cast<size_t>(K) * N * ea));
        VNPU_HIP(hipMalloc(&C, static_cast<size_t>(M) * N * 4));
        struct Free {
            void *a, *b, *c;
            ~Free() { (void)hipFree(a); (void)hipFree(b); (void)hipFree(c); }
        } freer{A, B, C};
        VNPU_HIP(hipMemset(A, 1, static_cast<size_t>(M) * K * ea));
        VNPU_HIP(hipMemset(B, 1, static_cast<size_t>(K) * N * ea));
        vnpu_packed_weights_t *w = nullptr;
        vnpu_command_t cmd{};
        if (i8) {
            w = pack_weights(device, static_cast<int8_t *>(B), nullptr, K, N, 0, 0);
            cmd.opcode = VNPU_OP_MATMUL_I8;
            cmd.args.matmul_i8.A = static_cast<int8_t *>(A);
            cmd.args.matmul_i8.B = w;
            cmd.args.matmul_i8.C = static_cast<float *>(C);
            cmd.args.matmul_i8.M = M;
            cmd.args.matmul_i8.K = K;
            cmd.args.matmul_i8.N = N;
        } else {
            cmd.opcode = VNPU_OP_MATMUL_F32;
            cmd.args.matmul_f32.A = static_cast<float *>(A);
            cmd.args.matmul_f32.B = static_cast<float *>(B);
            cmd.args.matmul_f32.C = static_cast<float *>(C);
            cmd.args.matmul_f32.M = M;
            cmd.args.matmul_f32.K = K;
            cmd.args.matmul_f32.N = N;
            cmd.args.matmul_f32.alpha = 1.0f;
        }
        struct Pack {
            vnpu_packed_weights_t *w;
            ~Pack() { if (w) destroy_packed(w); }
        } packguard{w};

        hipEvent_t e0, e1;
        VNPU_HIP(create_timing_event(&e0));
        VNPU_HIP(create_timing_event(&e1));
        auto time_tiles = [&](uint32_t tm, uint32_t tk, uint32_t tn, double &best) -> vnpu_status_t {
            apply_tiles(device, tm, tk, tn, which);
            vnpu_status_t r = vnpu_stream_submit(s, &cmd, 1, nullptr);   // warm-up
            if (r == VNPU_OK) r = vnpu_stream_sync(s);
            best = 1e30;
            for (uint32_t i = 0; r == VNPU_OK && i < iterations; ++i) {
                VNPU_HIP(hipEventRecord(e0, s->hip));
                r = vnpu_stream_submit(s, &cmd, 1, nullptr);
                VNPU_HIP(hipEventRecord(e1, s->hip));
                if (r == VNPU_OK) r = vnpu_stream_sync(s);
                float ms = 0.0f;
                VNPU_HIP(hipEventElapsedTime(&ms, e0, e1));
                best = std::min(best, static_cast<double>(ms));
            }
            return r;
        };
        struct Cand {
            uint32_t tm, tk, tn;
        };
        std::vector<Cand> cands;
        if (i8) {
            if (M % 256 == 0 && K % 128 == 0) cands.push_back({256, 128, 256});
            if (M % 256 == 0 && K % 128 == 0) cands.push_back({256, 128, 192});
            if (K % 128 == 0) cands.push_back({256, 128, 128});
            if (K % 64 == 0) cands.push_back({256, 64, 128});
            cands.push_back({128, 64, 128});
        } else {
            cands.push_back({128, (K + 15) / 16 * 16, 128});                 // no K split
            for (uint32_t d = (K / 2) / 16 * 16; d >= 64; d = (d / 2) / 16 * 16) cands.push_back({128, d, 128});
        }
        // The baseline is the kernel the device would run without the tune.
        double baseline = 0.0;
        {
            rc = vnpu_stream_submit(s, &cmd, 1, nullptr);
            if (rc == VNPU_OK) rc = vnpu_stream_sync(s);
            baseline = 1e30;
            for (uint32_t i = 0; rc == VNPU_OK && i < iterations; ++i) {
                VNPU_HIP(hipEventRecord(e0, s->hip));
                rc = vnpu_stream_submit(s, &cmd, 1, nullptr);
                VNPU_HIP(hipEventRecord(e1, s->hip));
                if (rc == VNPU_OK) rc = vnpu_stream_sync(s);
                float ms = 0.0f;
                VNPU_HIP(hipEventElapsedTime(&ms, e0, e1));
                baseline = std::min(baseline, static_cast<double>(ms));
            }
        }
        double best_ms = baseline;
        Cand best{orig_tm, orig_tk, orig_tn};
        bool improved = false;
        for (size_t i = 0; rc == VNPU_OK && i < cands.size(); ++i) {
            double ms = 0.0;
            rc = time_tiles(cands[i].tm, cands[i].tk, cands[i].tn, ms);
            if (rc == VNPU_OK && ms < best_ms) {
                best_ms = ms;
                best = cands[i];
                improved = true;
            }
        }
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        restore_tiles();
        if (rc != VNPU_OK) return rc;
        if (improved) apply_tiles(device, best.tm, best.tk, best.tn, which);
        result->tile_m = best.tm;
        result->tile_k = best.tk;
        result->tile_n = best.tn;
        result->unit = VNPU_UNIT_GPU;
        result->threads = device->cu_count;
        result->best_ms = best_ms;
        result->baseline_ms = baseline;
        result->speedup = best_ms > 0.0 ? baseline / best_ms : 0.0;
        result->gflops = 2.0 * M * K * N / (best_ms * 1e-3) * 1e-9;
        result->bytes_read = static_cast<uint64_t>(M) * K * 4 + static_cast<uint64_t>(K) * N * 4;
        result->bytes_written = static_cast<uint64_t>(M) * N * 4;
        return VNPU_OK;
    });
}

// The cluster client and the vnpu-node server are in cluster.cpp.

// ---------------------------------------------------------------------------
// Speculative step (reference src/cluster/cluster.cpp:552-646): draft gamma
// tokens one position at a time through draft_fn, score the gamma + 1
// positions with one verify_fn call, accept drafts while they equal the
// verifier's argmax (greedy acceptance, as the reference's v1), then sample a
// bonus token from the first rejected position.  The cluster handle is
// optional (no cluster is needed on one GPU).  The logits callbacks are the
// caller's; on this backend they would run MTP_HEAD_F32 / SOFTMAX_F32 on the
// GPU.  Sampling reproduces the reference's exactly: softmax weights from the
// same exp polynomial accumulated in double, one xorshift64 draw, the first
// index whose cumulative weight reaches u * sum.
// ---------------------------------------------------------------------------
namespace {

float host_fast_expf(float x)
{
    // The reference's 2^f polynomial (src/internal.h:87-108).  Unfused
    // multiply-then-add in each Horner step, as the reference's x86-64 build
    // evaluates it (no FMA in its target), so the sampling CDF and therefore
    // the sampled token agree bit for bit.
#pragma clang fp contract(off)
    if (x < -80.0f) return 0.0f;
    if (x > 80.0f) return std::numeric_limits<float>::infinity();
    const float z = x * 1.4426950408889634f;
    const float zi = std::floor(z);
    const float f = z - zi;
    float p = 0.0013333558146428443f;
    p = p * f + 0.009618129107628477f;
    p = p * f + 0.05550410866482158f;
    p = p * f + 0.2402265069591007f;
    p = p * f + 0.6931471805599453f;
    p = p * f + 1.0f;
    return std::ldexp(p, static_cast<int>(zi));
}

uint32_t argmax_finite(const float *logits, uint32_t vocab)
{
    uint32_t best = 0;
    float best_v = -std::numeric_limits<float>::infinity();
    for (uint32_t i = 0; i < vocab; ++i)
        if (std::isfinite(logits[i]) && logits[i] > best_v) {
            best_v = logits[i];
            best = i;
        }
    return best;
}

uint64_t next_xorshift64(uint64_t &state)
{
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    return state;
}

int32_t draw_token(const float *logits, uint32_t vocab, float temperature, uint64_t &rng)
{
    if (temperature <= 0.0f) return static_cast<int32_t>(argmax_finite(logits, vocab));
    float top = -std::numeric_limits<float>::infinity();
    for (uint32_t i = 0; i < vocab; ++i)
        if (std::isfinite(logits[i])) top = std::max(top, logits[i]);
    const float inv_t = 1.0f / temperature;
    std::vector<double> cum(vocab);
    double total = 0.0;
    for (uint32_t i = 0; i < vocab; ++i) {
        total += std::isfinite(logits[i]) ? host_fast_expf((logits[i] - top) * inv_t) : 0.0f;
        cum[i] = total;
    }
    if (total <= 0.0) return static_cast<int32_t>(argmax_finite(logits, vocab));
    const double u = static_cast<double>(next_xorshift64(rng) >> 11) / static_cast<double>(1ull << 53);
    const auto it = std::lower_bound(cum.begin(), cum.end(), u * total);
    return static_cast<int32_t>(std::min<size_t>(static_cast<size_t>(it - cum.begin()), vocab - 1));
}

}  // namespace

VNPU_API vnpu_status_t VNPU_CALL vnpu_speculative_step(vnpu_cluster_t *, const vnpu_speculative_config_t *config,
                                                       const int32_t *context, uint32_t context_len,
                                                       vnpu_logits_fn_t draft_fn, void *draft_user,
                                                       vnpu_logits_fn_t verify_fn, void *verify_user,
                                                       vnpu_speculative_result_t *result)
{
    if (!config || (!context && context_len) || !draft_fn || !verify_fn || !result || !config->vocab)
        return VNPU_ERR_INVALID_ARGUMENT;
    if (config->gamma == 0 || config->gamma >= VNPU_MAX_TOKENS) return VNPU_ERR_INVALID_ARGUMENT;
    return guard([&]() -> vnpu_status_t {
        std::memset(result, 0, sizeof(*result));
        const uint32_t gamma = config->gamma, vocab = config->vocab;
        std::vector<int32_t> seq(context, context + context_len);
        seq.reserve(context_len + gamma + 1);
        std::vector<int32_t> drafts(gamma);
        std::vector<float> logits(vocab);
        uint64_t rng = static_cast<uint64_t>(config->seed ? config->seed : 1) ^ 0x9e3779b97f4a7c15ull;
        const uint64_t t_begin = now_ns();
        for (uint32_t j = 0; j < gamma; ++j) {
            const vnpu_status_t rc = draft_fn(draft_user, seq.data(), static_cast<uint32_t>(seq.size()),
                                              context_len + j, 1, logits.data(), vocab);
            if (rc != VNPU_OK) return rc;
            drafts[j] = draw_token(logits.data(), vocab, config->temperature, rng);
            seq.push_back(drafts[j]);
        }
        const uint64_t t_drafted = now_ns();
        std::vector<float> scored(static_cast<size_t>(gamma + 1) * vocab, 0.0f);
        const vnpu_status_t rc = verify_fn(verify_user, seq.data(), static_cast<uint32_t>(seq.size()),
                                           context_len, gamma + 1, scored.data(), vocab);
        if (rc != VNPU_OK) return rc;
        const uint64_t t_verified = now_ns();
        uint32_t accepted = 0;
        while (accepted < gamma &&
               static_cast<int32_t>(argmax_finite(scored.data() + static_cast<size_t>(accepted) * vocab,
                                                  vocab)) == drafts[accepted])
            ++accepted;
        const int32_t bonus = draw_token(scored.data() + static_cast<size_t>(accepted) * vocab, vocab,
                                         config->temperature, rng);
        const uint32_t produced = accepted + 1;
        const uint32_t limit = config->max_tokens ? std::min(config->max_tokens, produced) : produced;
        for (uint32_t j = 0; j < limit; ++j) result->tokens[j] = j < accepted ? drafts[j] : bonus;
        result->accepted = std::min(accepted, limit);
        result->produced = limit;
        for (uint32_t j = 0; j < limit; ++j)
            if (result->tokens[j] == static_cast<int32_t>(config->eos_token)) {
                result->produced = j + 1;
                result->accepted = std::min(result->accepted, j + 1);
                result->eos = 1;
                break;
            }
        const double draft_ms = static_cast<double>(t_drafted - t_begin) / 1e6;
        const double verify_ms = static_cast<double>(t_verified - t_drafted) / 1e6;
        const double total_ms = static_cast<double>(now_ns() - t_begin) / 1e6;
        result->draft_time_ms = draft_ms;
        result->verify_time_ms = verify_ms;
        result->total_time_ms = total_ms;
        result->tokens_per_second = total_ms > 0.0 ? result->produced * 1000.0 / total_ms : 0.0;
        // produced tokens per (one verify + gamma drafts), in verify units
        result->theoretical_speedup =
            result->produced / (1.0 + gamma * (draft_ms / gamma) / std::max(verify_ms, 1e-6));
        return VNPU_OK;
    });
}

// ---------------------------------------------------------------------------
// Backend table (reference src/core/backend.cpp:8-60), same entry order.
// ---------------------------------------------------------------------------

static const vnpu_backend_v1_t g_backend_v1 = {
    VNPU_ABI_VERSION,
    sizeof(vnpu_backend_v1_t),
    "vnpu MI355X (gfx950 HIP)",
    vnpu_device_create,
    vnpu_device_destroy,
    vnpu_device_get_info,
    vnpu_device_get_status,
    vnpu_stream_create,
    vnpu_stream_destroy,
    vnpu_stream_sync,
    vnpu_stream_submit,
    vnpu_event_create,
    vnpu_event_destroy,
    vnpu_event_wait,
    vnpu_buffer_alloc,
    vnpu_buffer_free,
    vnpu_buffer_host_ptr,
    vnpu_matmul_f32,
    vnpu_matmul_i8,
    vnpu_quantize_i8,
    vnpu_pack_weights_i8,
    vnpu_packed_weights_destroy,
    vnpu_rmsnorm_f32,
    vnpu_softmax_f32,
    vnpu_rope_f32,
    vnpu_swiglu_f32,
    vnpu_gelu_f32,
    vnpu_attention_f32,
    vnpu_mtp_head_f32,
    vnpu_trace_enable,
    vnpu_trace_get_summary,
    vnpu_trace_dump,
    vnpu_trace_write_chrome,
    vnpu_autotune_gemm,
    vnpu_cluster_create,
    vnpu_cluster_destroy,
    vnpu_cluster_add_device,
    vnpu_cluster_add_remote,
    vnpu_cluster_cache_weights_f32,
    vnpu_cluster_matmul_f32,
    vnpu_cluster_get_stats,
    vnpu_node_run,
    vnpu_speculative_step,
    vnpu_status_string,
    vnpu_version_string,
    {}};

VNPU_API const vnpu_backend_v1_t *VNPU_CALL vnpu_get_backend_v1(void) { return &g_backend_v1; }

}  // extern "C"
