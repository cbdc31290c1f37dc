// dispatch.cpp - the vnpu command processor on a HIP stream.
//
// Replaces the reference's schedule_command and execute_* functions
// (src/core/scheduler.cpp:320-753).  For each vnpu_command_t it
//   1. validates arguments and applies the reference's defaults (same rules,
//      same rejections) - a rejected command throws ArgError, which the
//      stream turns into the reference's sticky-error behaviour;
//   2. stages host pointers through HBM (device pointers pass through);
//   3. picks the kernel from the shape (the "grid scheduler": int8 weight-
//      streaming GEMV below 64 rows, MFMA GEMM otherwise) and enqueues it on
//      the stream;
//   4. accounts algorithmic bytes / flops exactly as the reference does.
#include "vnpu_internal.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <tuple>

namespace vnpu {

namespace {
struct RangeRegistry {
    std::mutex mutex;
    std::map<uintptr_t, size_t> ranges;  // start -> bytes
};
RangeRegistry &ranges()
{
    static RangeRegistry *r = new RangeRegistry();
    return *r;
}
}  // namespace

void register_device_range(const void *p, size_t bytes)
{
    auto &r = ranges();
    std::lock_guard<std::mutex> lock(r.mutex);
    r.ranges[reinterpret_cast<uintptr_t>(p)] = bytes;
}

void unregister_device_range(const void *p)
{
    auto &r = ranges();
    std::lock_guard<std::mutex> lock(r.mutex);
    r.ranges.erase(reinterpret_cast<uintptr_t>(p));
}

bool is_device_pointer(const void *p)
{
    if (!p) return false;
    {
        auto &r = ranges();
        std::lock_guard<std::mutex> lock(r.mutex);
        const uintptr_t a = reinterpret_cast<uintptr_t>(p);
        auto it = r.ranges.upper_bound(a);
        if (it != r.ranges.begin()) {
            --it;
            if (a < it->first + it->second) return true;
        }
    }
    hipPointerAttribute_t attr;
    std::memset(&attr, 0, sizeof(attr));
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged ||
           attr.type == hipMemoryTypeUnified ||
           (attr.type == hipMemoryTypeHost && attr.devicePointer != nullptr);
}

namespace {

// Host-pointer staging for one command.  Device-accessible pointers are used
// as is; a pageable host pointer gets an HBM copy (in), a result copy-back
// (out) or both.  Any staging makes the command synchronous: pageable
// host copies are synchronous in HIP anyway.  The copies live in the
// stream's staging arena; a command needing more than it holds allocates the
// rest, and the arena grows to that size once the command has finished.
class Stager {
public:
    explicit Stager(hipStream_t s, vnpu_stream_t *owner = nullptr) : s_(s), owner_(owner) {}
    ~Stager() { release(); }

    template <typename T>
    const T *in(const T *p, size_t bytes)
    {
        if (!p || !bytes || is_device_pointer(p)) return p;
        void *d = alloc(bytes);
        VNPU_HIP(hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, s_));
        return static_cast<const T *>(d);
    }
    template <typename T>
    T *out(T *p, size_t bytes)
    {
        if (!p || !bytes || is_device_pointer(p)) return p;
        void *d = alloc(bytes);
        outs_.emplace_back(static_cast<void *>(p), d, bytes);
        return static_cast<T *>(d);
    }
    template <typename T>
    T *inout(T *p, size_t bytes)
    {
        if (!p || !bytes || is_device_pointer(p)) return p;
        void *d = alloc(bytes);
        VNPU_HIP(hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, s_));
        outs_.emplace_back(static_cast<void *>(p), d, bytes);
        return static_cast<T *>(d);
    }
    void finish()
    {
        for (auto &o : outs_)
            VNPU_HIP(hipMemcpyAsync(std::get<0>(o), std::get<1>(o), std::get<2>(o),
                                    hipMemcpyDeviceToHost, s_));
        outs_.clear();
        release();
    }

private:
    void *alloc(size_t bytes)
    {
        const size_t need = (bytes + 255) & ~static_cast<size_t>(255);
        total_ += need;
        if (owner_ && owner_->staging && used_ + need <= owner_->staging_bytes) {
            void *d = static_cast<char *>(owner_->staging) + used_;
            used_ += need;
            return d;
        }
        void *d = nullptr;
        VNPU_HIP(hipMalloc(&d, bytes));
        temps_.push_back(d);
        return d;
    }
    void release()
    {
        if (!total_) return;
        (void)hipStreamSynchronize(s_);
        for (void *d : temps_) (void)hipFree(d);
        temps_.clear();
        if (owner_ && total_ > owner_->staging_bytes) {
            // the stream is idle (synchronized above): replace the arena
            if (owner_->staging) (void)hipFree(owner_->staging);
            owner_->staging = nullptr;
            owner_->staging_bytes = 0;
            void *d = nullptr;
            if (hipMalloc(&d, total_) == hipSuccess) {
                owner_->staging = d;
                owner_->staging_bytes = total_;
            } else {
                (void)hipGetLastError();
            }
        }
        total_ = used_ = 0;
    }
    hipStream_t s_;
    vnpu_stream_t *owner_;
    size_t used_ = 0, total_ = 0;
    std::vector<void *> temps_;
    std::vector<std::tuple<void *, void *, size_t>> outs_;
};

inline void require(bool ok, const char *what)
{
    if (!ok) throw ArgError(what);
}

inline bool mul_overflow(uint64_t a, uint64_t b, uint64_t c)
{
    if (!a || !b || !c) return false;
    const uint64_t ab = a * b;
    if (ab / b != a) return true;
    return ab > std::numeric_limits<uint64_t>::max() / c;
}

// Bytes spanned by `rows` rows of `cols` elements at leading dimension ld.
inline size_t span(uint64_t rows, uint64_t cols, uint64_t ld, size_t elem)
{
    if (!rows || !cols) return 0;
    return static_cast<size_t>(((rows - 1) * ld + cols) * elem);
}

inline uint32_t cdiv(uint32_t a, uint32_t b) { return b ? (a + b - 1) / b : 0; }

// Range length of the reference's elementwise commands on a device of
// info.num_threads units (scheduler.cpp:541-543, 556-557, 569-570); each
// range has its own scalar tail, which SWIGLU and MUL round differently.
uint64_t ew_grain(const vnpu_device_t *dev, uint64_t count)
{
    const uint64_t units = std::max<uint32_t>(1, dev->info.num_threads);
    return std::max<uint64_t>(4096, count / (units * 4));
}

// choose_unit (reference scheduler.cpp:43-59).  UNIT_GPU is this backend's
// native unit and behaves like AUTO.
uint32_t choose_unit(uint32_t unit, bool has_mask, uint32_t flags)
{
    if (flags & VNPU_CMD_FLAG_CELL_DMA) return VNPU_UNIT_CELL;
    if (flags & VNPU_CMD_FLAG_VOODOO_FIFO) return VNPU_UNIT_VOODOO;
    if (unit != VNPU_UNIT_AUTO && unit != VNPU_UNIT_GPU) return unit;
    if (has_mask || (flags & VNPU_CMD_FLAG_WILDCAT_CULL)) return VNPU_UNIT_WILDCAT;
    return VNPU_UNIT_VOODOO;
}

bool pack_b_enabled()
{
    const char *e = std::getenv("VNPU_PACK");
    if (e && e[0] == '0' && e[1] == '\0') return false;
    const char *mode = std::getenv("VNPU_MODE");
    if (mode && std::strcmp(mode, "reference") == 0) return false;
    return true;
}

// The reference's f32 tile geometry (scheduler.cpp:96-206, the !int8
// branches), used only to sample a Wildcat cull mask so that the culled
// output region is the one the reference culls for the same device tiles and
// unit count.
void cull_geometry(const vnpu_device_t *dev, uint32_t unit, uint32_t M, uint32_t N, uint32_t &tm,
                   uint32_t &tn)
{
    tm = std::max<uint32_t>(1, dev->tile_m.load());
    tn = std::max<uint32_t>(1, dev->tile_n.load());
    const uint32_t units = std::max<uint32_t>(1, dev->info.num_threads);
    if (M <= 8 && (unit == VNPU_UNIT_VOODOO || unit == VNPU_UNIT_AUTO)) {
        tm = M;
        tn = std::min<uint32_t>(std::max<uint32_t>(32, tn), 64);
        if (tn > N) tn = N;
        return;
    }
    if (pack_b_enabled() && (unit == VNPU_UNIT_VOODOO || unit == VNPU_UNIT_AUTO)) {
        if (M >= 3 && cdiv(N, 64) >= 2 * units) {
            tm = M;
            tn = 64;
            return;
        }
    }
    if (unit == VNPU_UNIT_WILDCAT) {
        tm = std::min<uint32_t>(tm, 32);
        tn = std::min<uint32_t>(tn, 64);
    } else if (unit == VNPU_UNIT_CELL) {
        tm = std::min<uint32_t>(tm, 16);
        tn = std::min<uint32_t>(tn, 64);
    }
    uint64_t tiles = static_cast<uint64_t>(cdiv(M, tm)) * cdiv(N, tn);
    const uint64_t target = static_cast<uint64_t>(dev->info.num_threads) * 64;
    while (tiles > target && (tm < M || tn < N)) {
        if (tm < M) tm = std::min<uint32_t>(M, tm * 2);
        if (tn < N) tn = std::min<uint32_t>(N, tn * 2);
        tiles = static_cast<uint64_t>(cdiv(M, tm)) * cdiv(N, tn);
    }
}

// RoPE inverse-frequency table, computed on the host with the reference's
// expression 1 / powf(theta, 2j / dim) (llm.cpp:195-210) and cached per
// (theta, dim) in HBM for the device's lifetime.
struct InvFreqCache {
    std::mutex mutex;
    std::map<std::tuple<vnpu_device_t *, uint32_t, uint32_t>, float *> tables;
    ~InvFreqCache()
    {
        // Tables are released with their device (release_device_tables).
    }
};
InvFreqCache &inv_cache()
{
    static InvFreqCache *c = new InvFreqCache();
    return *c;
}

const float *rope_table(vnpu_device_t *dev, float theta, uint32_t dim)
{
    uint32_t bits;
    std::memcpy(&bits, &theta, 4);
    auto key = std::make_tuple(dev, bits, dim);
    auto &c = inv_cache();
    std::lock_guard<std::mutex> lock(c.mutex);
    auto it = c.tables.find(key);
    if (it != c.tables.end()) return it->second;
    const uint32_t half = dim / 2;
    std::vector<float> inv(half);
    for (uint32_t j = 0; j < half; ++j)
        inv[j] = 1.0f / std::pow(theta, 2.0f * static_cast<float>(j) / static_cast<float>(dim));
    float *d = nullptr;
    VNPU_HIP(hipMalloc(&d, half * sizeof(float)));
    VNPU_HIP(hipMemcpy(d, inv.data(), half * sizeof(float), hipMemcpyHostToDevice));
    c.tables.emplace(key, d);
    return d;
}

// RoPE cos/sin table: rows of (cos, sin) of (p * scaling) * inv[j] for the
// positions p = 0 .. rows-1, computed on the host with the C library's
// cosf / sinf - the very calls of the reference's rotate_vector
// (llm.cpp:195-211) - so the rotation is the reference's bit for bit.  One
// table per (device, theta, dim, scaling), grown to a power of two of
// positions as calls need more (at most kRopeMaxRows); a replaced table is
// kept until the device goes away, since kernels enqueued earlier may still
// read it.
constexpr uint32_t kRopeMaxRows = 65536;

struct RopeCs {
    float2 *table = nullptr;
    uint32_t rows = 0;
    std::vector<float2 *> retired;
};
struct RopeCsCache {
    std::mutex mutex;
    std::map<std::tuple<vnpu_device_t *, uint32_t, uint32_t, uint32_t>, RopeCs> tables;
};
RopeCsCache &rope_cs_cache()
{
    static RopeCsCache *c = new RopeCsCache();
    return *c;
}

const float2 *rope_cos_sin_table(vnpu_device_t *dev, float theta, uint32_t dim, float scaling, uint32_t need,
                                 uint32_t &rows)
{
    uint32_t tb, sb;
    std::memcpy(&tb, &theta, 4);
    std::memcpy(&sb, &scaling, 4);
    auto &c = rope_cs_cache();
    std::lock_guard<std::mutex> lock(c.mutex);
    RopeCs &t = c.tables[std::make_tuple(dev, tb, dim, sb)];
    need = std::min(need, kRopeMaxRows);
    if (need > t.rows) {
        uint32_t n = 64;
        while (n < need) n *= 2;
        n = std::min(n, kRopeMaxRows);
        const uint32_t half = dim / 2;
        std::vector<float> inv(half);
        for (uint32_t j = 0; j < half; ++j)
            inv[j] = 1.0f / std::pow(theta, 2.0f * static_cast<float>(j) / static_cast<float>(dim));
        std::vector<float2> host(static_cast<size_t>(n) * half);
        for (uint32_t p = 0; p < n; ++p) {
            const float pos = static_cast<float>(static_cast<int32_t>(p)) * scaling;
            for (uint32_t j = 0; j < half; ++j) {
                const float angle = pos * inv[j];
                host[static_cast<size_t>(p) * half + j] = make_float2(std::cos(angle), std::sin(angle));
            }
        }
        float2 *d = nullptr;
        VNPU_HIP(hipMalloc(&d, host.size() * sizeof(float2)));
        VNPU_HIP(hipMemcpy(d, host.data(), host.size() * sizeof(float2), hipMemcpyHostToDevice));
        if (t.table) t.retired.push_back(t.table);
        t.table = d;
        t.rows = n;
    }
    rows = t.rows;
    return t.table;
}

// ---------------------------------------------------------------------------

void exec_matmul_f32(vnpu_device_t *dev, vnpu_stream_t *s, const vnpu_matmul_f32_args_t &in,
                     uint32_t flags, ExecStats &st)
{
    // prepare_matmul_f32 (scheduler.cpp:274-318)
    require(in.A && in.B && in.C && in.M && in.K && in.N, "invalid matmul_f32 arguments");
    require(!mul_overflow(in.M, in.K, in.N), "matmul_f32 shape overflow");
    require(in.trans_a <= 1 && in.trans_b <= 1 && in.epilogue <= VNPU_EPILOGUE_GELU_ERF,
            "invalid matmul_f32 mode");
    const bool has_mask = in.tile_mask && in.mask_tile_m && in.mask_tile_n;
    const uint32_t unit = choose_unit(in.unit, in.tile_mask != nullptr, flags);
    st.unit = unit;
    k::F32Gemm p;
    p.M = in.M; p.K = in.K; p.N = in.N;
    p.lda = in.lda ? in.lda : (in.trans_a ? in.M : in.K);
    p.ldb = in.ldb ? in.ldb : (in.trans_b ? in.K : in.N);
    p.ldc = in.ldc ? in.ldc : in.N;
    require(p.lda >= (in.trans_a ? in.M : in.K) && p.ldb >= (in.trans_b ? in.K : in.N) &&
                p.ldc >= in.N,
            "invalid matmul_f32 leading dimensions");
    p.trans_a = in.trans_a;
    p.trans_b = in.trans_b;
    p.alpha = in.alpha == 0.0f ? 1.0f : in.alpha;
    p.beta = in.beta;
    p.epilogue = in.epilogue;
    // Device tiles 128 x depth x 128 (vnpu_device_set_tiles, an f32 autotune)
    // fix the K depth per workgroup; other tiles leave the choice automatic.
    p.k_split_depth = dev->f32_depth.load();
    p.err = s->err_dev;
    p.max_spin = dev->ws_max_spin;

    Stager sg(s->hip, s);
    p.A = sg.in(in.A, in.trans_a ? span(in.K, in.M, p.lda, 4) : span(in.M, in.K, p.lda, 4));
    p.B = sg.in(in.B, in.trans_b ? span(in.N, in.K, p.ldb, 4) : span(in.K, in.N, p.ldb, 4));
    p.bias = sg.in(in.bias, in.bias ? static_cast<size_t>(in.N) * 4 : 0);

    // Wildcat cull: sample the mask on the reference's tile grid, then
    // classify each 128 x 128 kernel tile as compute / culled / mixed.
    std::vector<uint8_t> cull, state;
    uint64_t culled_tiles = 0, total_tiles = 1;
    if (has_mask) {
        uint32_t tm, tn;
        cull_geometry(dev, unit, in.M, in.N, tm, tn);
        const uint32_t mt = cdiv(in.M, tm), nt = cdiv(in.N, tn);
        const uint8_t *mask = in.tile_mask;
        uint32_t bm, bn;
        k::gemm_f32_tile_dims(bm, bn);
        const uint32_t gm = cdiv(in.M, bm), gn = cdiv(in.N, bn);
        total_tiles = static_cast<uint64_t>(mt) * nt;
        p.cull_tm = tm;
        p.cull_tn = tn;
        p.cull_nt = nt;
        if (is_device_pointer(mask)) {
            // The mask may be written by earlier work on this stream: build
            // the cull map and tile states on the GPU, in stream order, and
            // count the culled tiles there (the status adds that count).
            {
                std::lock_guard<std::mutex> lock(dev->culled_mutex);
                if (!dev->culled_dev) {
                    void *c = nullptr;
                    VNPU_HIP(hipMalloc(&c, sizeof(unsigned long long)));
                    VNPU_HIP(hipMemset(c, 0, sizeof(unsigned long long)));
                    dev->culled_dev = static_cast<unsigned long long *>(c);
                }
            }
            const size_t cull_bytes = (total_tiles + 255) / 256 * 256;
            uint8_t *scratch = static_cast<uint8_t *>(
                s->ensure_cull_scratch(cull_bytes + static_cast<size_t>(gm) * gn));
            k::cull_classify(s->hip, mask, in.mask_tile_m, in.mask_tile_n, in.M, in.N, tm, tn, scratch,
                             scratch + cull_bytes, dev->culled_dev);
            p.cull = scratch;
            p.ktile_state = scratch + cull_bytes;
        }
    }
    if (has_mask && p.cull == nullptr) {   // a host mask: classified here
        const uint32_t mt = cdiv(in.M, p.cull_tm), nt = p.cull_nt;
        const uint32_t tm = p.cull_tm, tn = p.cull_tn;
        const uint8_t *mask = in.tile_mask;
        cull.assign(static_cast<size_t>(mt) * nt, 0);
        for (uint32_t mi = 0; mi < mt; ++mi)
            for (uint32_t ni = 0; ni < nt; ++ni) {
                const uint32_t mm = std::min<uint32_t>(in.mask_tile_m - 1,
                    static_cast<uint32_t>((static_cast<uint64_t>(mi) * in.mask_tile_m) / mt));
                const uint32_t nn = std::min<uint32_t>(in.mask_tile_n - 1,
                    static_cast<uint32_t>((static_cast<uint64_t>(ni) * in.mask_tile_n) / nt));
                if (mask[static_cast<size_t>(mm) * in.mask_tile_n + nn] == 0) {
                    cull[static_cast<size_t>(mi) * nt + ni] = 1;
                    ++culled_tiles;
                }
            }
        uint32_t bm, bn;
        k::gemm_f32_tile_dims(bm, bn);
        const uint32_t gm = cdiv(in.M, bm), gn = cdiv(in.N, bn);
        state.assign(static_cast<size_t>(gm) * gn, 0);
        for (uint32_t gi = 0; gi < gm; ++gi)
            for (uint32_t gj = 0; gj < gn; ++gj) {
                const uint32_t r0 = gi * bm / tm, r1 = (std::min(in.M, (gi + 1) * bm) - 1) / tm;
                const uint32_t c0 = gj * bn / tn, c1 = (std::min(in.N, (gj + 1) * bn) - 1) / tn;
                bool any_c = false, any_k = false;
                for (uint32_t r = r0; r <= r1; ++r)
                    for (uint32_t c = c0; c <= c1; ++c)
                        (cull[static_cast<size_t>(r) * nt + c] ? any_c : any_k) = true;
                state[static_cast<size_t>(gi) * gn + gj] = any_c ? (any_k ? 2 : 1) : 0;
            }
        p.cull = sg.in(cull.data(), cull.size());
        p.ktile_state = sg.in(state.data(), state.size());
        // A host vector always stages; keep them alive until finish().
    }
    const bool c_in = in.beta != 0.0f || p.ldc != in.N;
    const size_t c_bytes = span(in.M, in.N, p.ldc, 4);
    p.C = c_in ? sg.inout(in.C, c_bytes) : sg.out(in.C, c_bytes);

    if (!has_mask && in.M <= 8 && !in.trans_a && !in.trans_b && k::gemv_f32_supported(p)) {
        const size_t ws = k::gemv_f32_ws_bytes(p);
        float *w = static_cast<float *>(s->ensure_workspace(ws));
        k::gemv_f32(s->hip, p, w);
    } else {
        const size_t ws = k::gemm_f32_ws_bytes(p);
        k::gemm_f32(s->hip, p, ws ? static_cast<float *>(s->ensure_workspace(ws)) : nullptr);
    }
    VNPU_HIP(hipGetLastError());
    sg.finish();

    st.tiles_dispatched += total_tiles - culled_tiles;
    st.tiles_culled += culled_tiles;
    const uint64_t a_b = static_cast<uint64_t>(in.M) * in.K * 4;
    const uint64_t b_b = static_cast<uint64_t>(in.K) * in.N * 4;
    const uint64_t c_b = static_cast<uint64_t>(in.M) * in.N * 4;
    const uint64_t bias_b = in.bias ? static_cast<uint64_t>(in.N) * 4 : 0;
    st.bytes_read += a_b + b_b + bias_b + (in.beta != 0.0f ? c_b : 0);
    st.bytes_written += c_b;
    st.flops += 2ull * in.M * in.K * in.N;
}

void exec_matmul_i8(vnpu_device_t *dev, vnpu_stream_t *s, const vnpu_matmul_i8_args_t &in,
                    uint32_t flags, ExecStats &st)
{
    // execute_matmul_i8 (scheduler.cpp:370-428)
    vnpu_packed_weights_t *w = in.B;
    require(in.A && w && in.C && in.M && in.K && in.N, "invalid matmul_i8 arguments");
    require(w->K == in.K && w->N == in.N, "packed weight shape mismatch");
    require(w->device == nullptr || w->device->hip_device == dev->hip_device,
            "packed weights live on another device");
    st.unit = choose_unit(in.unit, false, flags);
    k::I8Gemm p;
    p.M = in.M; p.N = in.N; p.K = in.K;
    p.lda = in.lda ? in.lda : in.K;
    p.ldc = in.ldc ? in.ldc : in.N;
    require(p.lda >= in.K && p.ldc >= in.N, "invalid int8 leading dimensions");
    p.frag = w->frag;
    p.Kp = w->Kp;
    p.Np = w->Np;
    p.nz_list = w->nz_list;
    p.nz_count = w->nz_count;
    p.nz_tiles = w->nz_tiles;
    p.scale_b = w->scales_dev;
    p.epilogue = in.epilogue;
    p.variant = dev->i8_variant.load();
    require(in.epilogue <= VNPU_EPILOGUE_GELU_ERF, "invalid matmul_i8 epilogue");

    Stager sg(s->hip, s);
    p.A = sg.in(in.A, span(in.M, in.K, p.lda, 1));
    p.scale_a = sg.in(in.scale_a, in.scale_a ? static_cast<size_t>(in.M) * 4 : 0);
    p.bias = sg.in(in.bias, in.bias ? static_cast<size_t>(in.N) * 4 : 0);
    const size_t c_bytes = span(in.M, in.N, p.ldc, 4);
    p.C = p.ldc != in.N ? sg.inout(in.C, c_bytes) : sg.out(in.C, c_bytes);

    if (k::gemv_i8_takes(in.M, in.N))
        k::gemv_i8(s->hip, p);
    else
        k::gemm_i8(s->hip, p, static_cast<int8_t *>(s->ensure_workspace(k::gemm_i8_ws_bytes(p))));
    VNPU_HIP(hipGetLastError());
    sg.finish();

    st.tiles_dispatched += 1;
    const uint64_t a_b = static_cast<uint64_t>(in.M) * in.K;
    const uint64_t b_b = static_cast<uint64_t>(in.K) * in.N;
    const uint64_t c_b = static_cast<uint64_t>(in.M) * in.N * 4;
    const uint64_t sc_b = static_cast<uint64_t>(in.N + (in.scale_a ? in.M : 0)) * 4;
    st.bytes_read += a_b + b_b + sc_b;
    st.bytes_written += c_b;
    st.flops += 2ull * in.M * in.K * in.N;
}

}  // namespace

// Two MATMUL_I8 commands in a row, on device-resident data, with the same M
// and neither reading nor writing what the other writes (the block's gate and
// up projections): one wide-tile grid when that runs fewer whole rounds of
// tiles (k::gemm_i8_pair), or at M <= 8 one matrix-core GEMV grid
// (k::gemv_i8_pair).  Returns false, having launched nothing, when the pair
// does not qualify; the commands then run one by one as usual.
bool try_execute_pair(vnpu_device_t *dev, vnpu_stream_t *s, const vnpu_command_t &c0,
                      const vnpu_command_t &c1, uint32_t flags, ExecStats &st0, ExecStats &st1)
{
    if (c0.opcode != VNPU_OP_MATMUL_I8 || c1.opcode != VNPU_OP_MATMUL_I8) return false;
    const vnpu_matmul_i8_args_t *in[2] = {&c0.args.matmul_i8, &c1.args.matmul_i8};
    k::I8Gemm p[2];
    struct Range {
        uintptr_t lo = 0, hi = 0;
        bool overlaps(const Range &o) const { return lo < o.hi && o.lo < hi; }
    };
    Range ra[2], rc[2], rs[2], rb[2];
    const uint32_t variant = dev->i8_variant.load();
    for (int i = 0; i < 2; ++i) {
        const vnpu_matmul_i8_args_t &a = *in[i];
        const vnpu_packed_weights_t *w = a.B;
        if (!a.A || !w || !a.C || !a.M || !a.K || !a.N || (a.M <= 8) != (in[0]->M <= 8)) return false;
        if (w->K != a.K || w->N != a.N || a.epilogue > VNPU_EPILOGUE_GELU_ERF) return false;
        if (w->device && w->device->hip_device != dev->hip_device) return false;
        const uint32_t lda = a.lda ? a.lda : a.K, ldc = a.ldc ? a.ldc : a.N;
        if (lda < a.K || ldc < a.N) return false;
        if (!is_device_pointer(a.A) || !is_device_pointer(a.C) || (a.scale_a && !is_device_pointer(a.scale_a)) ||
            (a.bias && !is_device_pointer(a.bias)))
            return false;
        k::I8Gemm &q = p[i];
        q.A = a.A; q.lda = lda; q.frag = w->frag;
        q.Kp = w->Kp; q.Np = w->Np; q.scale_a = a.scale_a; q.scale_b = w->scales_dev; q.bias = a.bias;
        q.C = a.C; q.ldc = ldc; q.M = a.M; q.N = a.N; q.K = a.K; q.epilogue = a.epilogue; q.variant = variant;
        auto range = [](const void *ptr, size_t bytes) {
            Range r;
            r.lo = reinterpret_cast<uintptr_t>(ptr);
            r.hi = r.lo + bytes;
            return r;
        };
        ra[i] = range(a.A, span(a.M, a.K, lda, 1));
        rc[i] = range(a.C, span(a.M, a.N, ldc, 4));
        rs[i] = a.scale_a ? range(a.scale_a, static_cast<size_t>(a.M) * 4) : Range{};
        rb[i] = a.bias ? range(a.bias, static_cast<size_t>(a.N) * 4) : Range{};
    }
    for (int i = 0; i < 2; ++i) {
        const int o = 1 - i;
        if (rc[i].overlaps(ra[o]) || rc[i].overlaps(rs[o]) || rc[i].overlaps(rb[o]) || rc[i].overlaps(rc[o]))
            return false;
    }
    if (!(in[0]->M <= 8 ? k::gemv_i8_pair(s->hip, p[0], p[1]) : k::gemm_i8_pair(s->hip, p[0], p[1])))
        return false;
    VNPU_HIP(hipGetLastError());
    ExecStats *st[2] = {&st0, &st1};
    for (int i = 0; i < 2; ++i) {
        const vnpu_matmul_i8_args_t &a = *in[i];
        st[i]->unit = choose_unit(a.unit, false, flags);
        st[i]->tiles_dispatched += 1;
        st[i]->bytes_read += static_cast<uint64_t>(a.M) * a.K + static_cast<uint64_t>(a.K) * a.N +
                             static_cast<uint64_t>(a.N + (a.scale_a ? a.M : 0)) * 4;
        st[i]->bytes_written += static_cast<uint64_t>(a.M) * a.N * 4;
        st[i]->flops += 2ull * a.M * a.K * a.N;
    }
    return true;
}

// MATMUL_I8 at M <= 8 followed by an ADD_F32 of its output (the block's
// down projection + residual at decode): the GEMV's store also writes the
// ADD's result, one launch instead of two.  Device-resident buffers, C
// contiguous, the ADD over exactly C's M x N elements with C as one operand;
// its output may be the other operand (in place) or C itself, and must not
// overlap anything else the GEMV reads.  Returns false, having launched
// nothing, when the pair does not qualify.
bool try_execute_matmul_add(vnpu_device_t *dev, vnpu_stream_t *s, const vnpu_command_t &c0,
                            const vnpu_command_t &c1, uint32_t flags, ExecStats &st0, ExecStats &st1)
{
    if (c0.opcode != VNPU_OP_MATMUL_I8 || c1.opcode != VNPU_OP_ADD_F32) return false;
    const vnpu_matmul_i8_args_t &in = c0.args.matmul_i8;
    const vnpu_binary_f32_args_t &ad = c1.args.binary;
    const vnpu_packed_weights_t *w = in.B;
    if (!in.A || !w || !in.C || !in.M || !in.K || !in.N || in.M > 8) return false;
    if (w->K != in.K || w->N != in.N || in.epilogue > VNPU_EPILOGUE_GELU_ERF) return false;
    if (w->device && w->device->hip_device != dev->hip_device) return false;
    const uint32_t lda = in.lda ? in.lda : in.K;
    if (lda < in.K || (in.ldc && in.ldc != in.N)) return false;
    const uint64_t count = static_cast<uint64_t>(in.M) * in.N;
    if (ad.count != count || !ad.Y || (ad.A == in.C) == (ad.B == in.C)) return false;
    const bool c_first = ad.A == in.C;
    const float *res = c_first ? ad.B : ad.A;
    if (!res) return false;
    for (const void *q : {static_cast<const void *>(in.A), static_cast<const void *>(in.C),
                          static_cast<const void *>(in.scale_a), static_cast<const void *>(in.bias),
                          static_cast<const void *>(res), static_cast<const void *>(ad.Y)})
        if (q && !is_device_pointer(q)) return false;
    auto lo = [](const void *q) { return reinterpret_cast<uintptr_t>(q); };
    auto overlaps = [&](const void *a, size_t an, const void *b, size_t bn) {
        return a && b && lo(a) < lo(b) + bn && lo(b) < lo(a) + an;
    };
    const size_t fb = count * 4;
    // C and the other operand: disjoint (each is read or written once per element)
    if (overlaps(in.C, fb, res, fb)) return false;
    // Y: exactly the other operand or C, or disjoint from both; never over the GEMV's inputs
    if (ad.Y != res && overlaps(ad.Y, fb, res, fb)) return false;
    if (ad.Y != in.C && overlaps(ad.Y, fb, in.C, fb)) return false;
    if (overlaps(ad.Y, fb, in.A, span(in.M, in.K, lda, 1)) ||
        overlaps(ad.Y, fb, in.scale_a, in.scale_a ? static_cast<size_t>(in.M) * 4 : 0) ||
        overlaps(ad.Y, fb, in.bias, in.bias ? static_cast<size_t>(in.N) * 4 : 0) ||
        overlaps(in.C, fb, in.A, span(in.M, in.K, lda, 1)))
        return false;

    k::I8Gemm p;
    p.A = in.A; p.lda = lda; p.frag = w->frag;
    p.Kp = w->Kp; p.Np = w->Np; p.scale_a = in.scale_a; p.scale_b = w->scales_dev; p.bias = in.bias;
    p.nz_list = w->nz_list; p.nz_count = w->nz_count; p.nz_tiles = w->nz_tiles;
    p.C = in.C; p.ldc = in.N; p.M = in.M; p.N = in.N; p.K = in.K; p.epilogue = in.epilogue;
    p.variant = dev->i8_variant.load();
    const bool both0 = ad.alpha == 0.0f && ad.beta == 0.0f;  // llm.cpp:226-227
    p.res = res;
    p.res_out = ad.Y;
    p.res_alpha = both0 ? 1.0f : ad.alpha;
    p.res_beta = both0 ? 1.0f : ad.beta;
    p.res_c_first = c_first ? 1u : 0u;
    k::gemv_i8(s->hip, p);
    VNPU_HIP(hipGetLastError());

    st0.unit = choose_unit(in.unit, false, flags);
    st0.tiles_dispatched += 1;
    st0.bytes_read += static_cast<uint64_t>(in.M) * in.K + static_cast<uint64_t>(in.K) * in.N +
                      static_cast<uint64_t>(in.N + (in.scale_a ? in.M : 0)) * 4;
    st0.bytes_written += count * 4;
    st0.flops += 2ull * in.M * in.K * in.N;
    st1.bytes_read += count * 8;
    st1.bytes_written += count * 4;
    st1.flops += count * 3;
    return true;
}

uint32_t try_execute_chain(vnpu_stream_t *s, const vnpu_command_t *c, uint64_t n,
                           uint32_t *matched, ExecStats *st)
{
    *matched = 0;
    if (n < 2) return 0;
    k::RowChain p;
    uint32_t used = 0;
    const vnpu_rmsnorm_f32_args_t *norm = nullptr;
    const vnpu_quantize_i8_args_t *quant = nullptr;
    uint64_t pre_count = 0;
    const uint32_t op0 = c[0].opcode;
    if (op0 == VNPU_OP_ADD_F32 || op0 == VNPU_OP_SWIGLU_F32) {
        if (op0 == VNPU_OP_ADD_F32) {
            const auto &a = c[0].args.binary;  // scheduler.cpp:564-581
            const bool both0 = a.alpha == 0.0f && a.beta == 0.0f;
            p.pre = k::kChainAdd;
            p.A = a.A; p.B = a.B; p.Y = a.Y; pre_count = a.count;
            p.alpha = both0 ? 1.0f : a.alpha;
            p.beta = both0 ? 1.0f : a.beta;
            if (c[1].opcode != VNPU_OP_RMSNORM_F32 || c[1].args.rmsnorm.X != a.Y) return 0;
            norm = &c[1].args.rmsnorm;
            used = 2;
            if (n > 2 && c[2].opcode == VNPU_OP_QUANTIZE_I8) {
                quant = &c[2].args.quantize_i8;
                used = 3;
            }
        } else {
            const auto &a = c[0].args.swiglu;  // scheduler.cpp:536-548
            p.pre = k::kChainSwiglu;
            p.A = a.gate; p.B = a.up; p.Y = a.Y; pre_count = a.count;
            p.alpha = a.alpha == 0.0f ? 1.0f : a.alpha;
            if (c[1].opcode != VNPU_OP_QUANTIZE_I8 || c[1].args.quantize_i8.X != a.Y) return 0;
            quant = &c[1].args.quantize_i8;
            used = 2;
        }
        if (!p.A || !p.B || !p.Y || !pre_count) return 0;
    } else if (op0 == VNPU_OP_RMSNORM_F32) {
        if (c[1].opcode != VNPU_OP_QUANTIZE_I8) return 0;
        norm = &c[0].args.rmsnorm;
        quant = &c[1].args.quantize_i8;
        p.A = norm->X;
        used = 2;
    } else {
        return 0;
    }
    if (norm) {
        if (!norm->X || !norm->Y || !norm->rows || !norm->cols) return 0;  // scheduler.cpp:475-492
        p.rows = norm->rows;
        p.cols = norm->cols;
        p.W = norm->W;
        p.Nrm = norm->Y;
        p.eps = norm->eps > 0.0f ? norm->eps : 1e-5f;
    }
    if (quant) {
        const float *qx = norm ? norm->Y : p.Y;
        if (quant->X != qx || !quant->Y || !quant->scales || quant->axis != VNPU_QUANT_PER_ROW ||
            !quant->rows || !quant->cols || quant->rows > 0xffffffffull || quant->cols > 0xffffffffull)
            quant = nullptr;
        else if (norm && (quant->rows != norm->rows || quant->cols != norm->cols))
            quant = nullptr;
        if (!quant) {
            if (op0 != VNPU_OP_ADD_F32) return 0;
            used = 2;  // ADD -> RMSNORM without the quantize
        } else {
            p.rows = static_cast<uint32_t>(quant->rows);
            p.cols = static_cast<uint32_t>(quant->cols);
            p.Q = quant->Y;
            p.scales = quant->scales;
        }
    }
    const uint64_t elems = static_cast<uint64_t>(p.rows) * p.cols;
    if (pre_count && pre_count != elems) return 0;
    p.grain = ew_grain(s->device, elems);

    // Aliasing: every output must be disjoint from every other buffer of the
    // chain, except that float rows (A, B, Y, Nrm) may be the same buffer;
    // then each workgroup reads its row before writing it and the result is
    // the one of the commands run in order.
    struct Buf {
        const void *p;
        size_t bytes;
        bool row, out;
    };
    const size_t rb = elems * 4;
    Buf bufs[7];
    int nb = 0;
    auto add = [&](const void *q, size_t bytes, bool row, bool out) {
        if (q) bufs[nb++] = Buf{q, bytes, row, out};
    };
    add(p.A, rb, true, false);
    add(p.B, rb, true, false);
    add(p.Y, rb, true, true);
    add(p.W, static_cast<size_t>(p.cols) * 4, false, false);
    add(p.Nrm, rb, true, true);
    add(p.Q, elems, false, true);
    add(p.scales, static_cast<size_t>(p.rows) * 4, false, true);
    for (int i = 0; i < nb; ++i) {
        if (!is_device_pointer(bufs[i].p)) return 0;
        if (!bufs[i].out) continue;
        const uintptr_t lo = reinterpret_cast<uintptr_t>(bufs[i].p), hi = lo + bufs[i].bytes;
        for (int j = 0; j < nb; ++j) {
            if (j == i) continue;
            const uintptr_t lo2 = reinterpret_cast<uintptr_t>(bufs[j].p), hi2 = lo2 + bufs[j].bytes;
            if (lo < hi2 && lo2 < hi && !(bufs[i].row && bufs[j].row && lo == lo2)) return 0;
        }
    }

    *matched = used;
    if (!k::row_chain(s->hip, p)) {
        *matched = 0;
        return 0;
    }
    VNPU_HIP(hipGetLastError());
    // Per-command accounting as the unfused commands count it.
    uint32_t slot = 0;
    if (p.pre == k::kChainAdd) {
        st[slot].bytes_read += elems * 8;
        st[slot].bytes_written += elems * 4;
        st[slot++].flops += elems * 3;
    } else if (p.pre == k::kChainSwiglu) {
        st[slot].bytes_read += elems * 8;
        st[slot].bytes_written += elems * 4;
        st[slot++].flops += elems * 8;
    }
    if (p.Nrm) {
        st[slot].bytes_read += elems * 4 + (p.W ? static_cast<uint64_t>(p.cols) * 4 : 0);
        st[slot].bytes_written += elems * 4;
        st[slot++].flops += elems * 5;
    }
    if (p.Q) {
        st[slot].bytes_read += elems * 4;
        st[slot].bytes_written += elems;
        st[slot++].flops += elems * 3;
    }
    return used;
}

namespace {

void exec_quantize(vnpu_device_t *, vnpu_stream_t *s, const vnpu_quantize_i8_args_t &a,
                   ExecStats &st)
{
    // execute_quantize_i8 (scheduler.cpp:430-473)
    require(a.X && a.Y && a.scales && a.rows && a.cols && a.axis <= VNPU_QUANT_PER_TENSOR,
            "invalid quantize_i8 arguments");
    require(!mul_overflow(a.rows, a.cols, 1), "quantize shape overflow");
    const uint64_t total = a.rows * a.cols;
    const size_t n_scales = a.axis == VNPU_QUANT_PER_ROW ? a.rows
                            : a.axis == VNPU_QUANT_PER_COLUMN ? a.cols : 1;
    Stager sg(s->hip, s);
    const float *X = sg.in(a.X, total * 4);
    int8_t *Y = sg.out(a.Y, total);
    float *sc = sg.out(a.scales, n_scales * 4);
    if (a.axis == VNPU_QUANT_PER_ROW) {
        k::quantize_rows(s->hip, X, Y, sc, a.rows, a.cols);
    } else if (a.axis == VNPU_QUANT_PER_COLUMN) {
        require(a.cols <= 0xffffffffull * 256ull, "quantize column count too large");
        uint32_t *ws = static_cast<uint32_t *>(s->ensure_workspace(k::quantize_cols_ws_bytes(a.cols)));
        k::quantize_cols(s->hip, X, Y, sc, a.rows, a.cols, ws);
    } else {
        float *ws = static_cast<float *>(s->ensure_workspace(k::quantize_tensor_ws_bytes()));
        k::quantize_tensor(s->hip, X, Y, sc, total, ws);
    }
    VNPU_HIP(hipGetLastError());
    sg.finish();
    st.bytes_read += total * 4;
    st.bytes_written += total;
    st.flops += total * 3;
}

void exec_rmsnorm(vnpu_stream_t *s, const vnpu_rmsnorm_f32_args_t &a, ExecStats &st)
{
    // execute_rmsnorm (scheduler.cpp:475-492), eps default llm.cpp:67
    require(a.X && a.Y && a.rows && a.cols, "invalid rmsnorm arguments");
    const float eps = a.eps > 0.0f ? a.eps : 1e-5f;
    const uint64_t n = static_cast<uint64_t>(a.rows) * a.cols;
    Stager sg(s->hip, s);
    const float *X = sg.in(a.X, n * 4);
    const float *W = sg.in(a.W, a.W ? static_cast<size_t>(a.cols) * 4 : 0);
    float *Y = (a.Y == a.X) ? sg.inout(a.Y, n * 4) : sg.out(a.Y, n * 4);
    if (a.Y == a.X && !is_device_pointer(a.X)) X = Y;
    k::rmsnorm(s->hip, X, W, Y, a.rows, a.cols, eps);
    VNPU_HIP(hipGetLastError());
    sg.finish();
    st.bytes_read += n * 4 + (a.W ? static_cast<uint64_t>(a.cols) * 4 : 0);
    st.bytes_written += n * 4;
    st.flops += n * 5;
}

void exec_softmax(vnpu_stream_t *s, const vnpu_softmax_f32_args_t &a, ExecStats &st)
{
    // execute_softmax (scheduler.cpp:494-510), temperature default llm.cpp:119
    require(a.X && a.Y && a.rows && a.cols, "invalid softmax arguments");
    const float inv_t = a.temperature > 0.0f ? 1.0f / a.temperature : 1.0f;
    const uint64_t n = static_cast<uint64_t>(a.rows) * a.cols;
    Stager sg(s->hip, s);
    const float *X = sg.in(a.X, n * 4);
    float *Y = (a.Y == a.X) ? sg.inout(a.Y, n * 4) : sg.out(a.Y, n * 4);
    if (a.Y == a.X && !is_device_pointer(a.X)) X = Y;
    const size_t ws_bytes = k::softmax_ws_bytes(a.rows, a.cols);
    float *ws = ws_bytes ? static_cast<float *>(s->ensure_workspace(ws_bytes)) : nullptr;
    k::softmax(s->hip, X, Y, a.rows, a.cols, inv_t, ws);
    VNPU_HIP(hipGetLastError());
    sg.finish();
    st.bytes_read += n * 4;
    st.bytes_written += n * 4;
    st.flops += n * 6;
}

void exec_rope(vnpu_device_t *dev, vnpu_stream_t *s, const vnpu_rope_f32_args_t &a, ExecStats &st)
{
    // execute_rope (scheduler.cpp:512-534), defaults llm.cpp:583-584
    require((a.Q || a.K) && a.batch && a.heads && a.head_dim && (a.q_seq || a.k_seq) &&
                !(a.head_dim & 1u),
            "invalid rope arguments");
    const float theta = a.theta_base > 0.0f ? a.theta_base : 10000.0f;
    const float scaling = a.scaling > 0.0f ? a.scaling : 1.0f;
    const uint64_t bh = static_cast<uint64_t>(a.batch) * a.heads;
    const uint64_t qn = bh * a.q_seq * a.head_dim, kn = bh * a.k_seq * a.head_dim;
    const uint32_t seq = std::max(a.q_seq, a.k_seq);
    const float *inv = rope_table(dev, theta, a.head_dim);
    // Positions the table must cover: known on the host for offset-based
    // positions and host position arrays; a device position array uses the
    // rows the table already has (other positions compute cos/sin on the GPU).
    uint64_t need = 0;
    if (!a.positions) {
        need = static_cast<uint64_t>(a.position_offset) + seq;
    } else if (!is_device_pointer(a.positions)) {
        for (uint32_t t = 0; t < seq; ++t)
            if (a.positions[t] >= 0) need = std::max<uint64_t>(need, static_cast<uint64_t>(a.positions[t]) + 1);
    }
    uint32_t cs_rows = 0;
    const float2 *cs = rope_cos_sin_table(dev, theta, a.head_dim, scaling,
                                          static_cast<uint32_t>(std::min<uint64_t>(need, kRopeMaxRows)), cs_rows);
    Stager sg(s->hip, s);
    float *Q = a.Q && a.q_seq ? sg.inout(a.Q, qn * 4) : nullptr;
    float *K = a.K && a.k_seq ? sg.inout(a.K, kn * 4) : nullptr;
    const int32_t *pos = sg.in(a.positions, a.positions ? static_cast<size_t>(seq) * 4 : 0);
    k::rope(s->hip, Q, K, pos, a.batch, a.heads, Q ? a.q_seq : 0, K ? a.k_seq : 0, a.head_dim,
            a.position_offset, a.interleaved, scaling, inv, cs, cs_rows);
    VNPU_HIP(hipGetLastError());
    sg.finish();
    st.bytes_read += (qn + kn) * 4;
    st.bytes_written += (qn + kn) * 4;
    st.flops += (qn + kn) * 8;
}

void exec_elementwise(vnpu_stream_t *s, const vnpu_command_t &cmd, ExecStats &st)
{
    Stager sg(s->hip, s);
    if (cmd.opcode == VNPU_OP_SWIGLU_F32) {
        const auto &a = cmd.args.swiglu;  // scheduler.cpp:536-548
        require(a.gate && a.up && a.Y && a.count, "invalid swiglu arguments");
        const float alpha = a.alpha == 0.0f ? 1.0f : a.alpha;
        const float *g = sg.in(a.gate, a.count * 4);
        const float *u = sg.in(a.up, a.count * 4);
        float *Y = sg.out(a.Y, a.count * 4);
        k::swiglu(s->hip, g, u, Y, a.count, alpha, ew_grain(s->device, a.count));
        st.bytes_read += a.count * 8;
        st.bytes_written += a.count * 4;
        st.flops += a.count * 8;
    } else if (cmd.opcode == VNPU_OP_GELU_F32) {
        const auto &a = cmd.args.unary;  // scheduler.cpp:550-562
        require(a.X && a.Y && a.count, "invalid gelu arguments");
        const float *X = sg.in(a.X, a.count * 4);
        float *Y = sg.out(a.Y, a.count * 4);
        k::gelu(s->hip, X, Y, a.count);
        st.bytes_read += a.count * 4;
        st.bytes_written += a.count * 4;
        st.flops += a.count * 12;
    } else {
        const auto &a = cmd.args.binary;  // scheduler.cpp:564-581
        require(a.A && a.B && a.Y && a.count, "invalid binary arguments");
        const float *A = sg.in(a.A, a.count * 4);
        const float *B = sg.in(a.B, a.count * 4);
        float *Y = sg.out(a.Y, a.count * 4);
        if (cmd.opcode == VNPU_OP_ADD_F32) {
            const bool both0 = a.alpha == 0.0f && a.beta == 0.0f;  // llm.cpp:226-227
            k::add(s->hip, A, B, Y, a.count, both0 ? 1.0f : a.alpha, both0 ? 1.0f : a.beta);
        } else {
            k::mul(s->hip, A, B, Y, a.count, a.alpha == 0.0f ? 1.0f : a.alpha, a.beta,
                   ew_grain(s->device, a.count));
        }
        st.bytes_read += a.count * 8;
        st.bytes_written += a.count * 4;
        st.flops += a.count * 3;
    }
    VNPU_HIP(hipGetLastError());
    sg.finish();
}

// execute_attention (scheduler.cpp:583-608), scale default llm.cpp:452-453:
// validation and the kernel parameters, pointers left to the caller.
k::Attn attention_params(const vnpu_attention_f32_args_t &a)
{
    require(a.Q && a.K && a.V && a.O && a.batch && a.heads && a.seq_q && a.seq_k && a.head_dim,
            "invalid attention arguments");
    k::Attn p;
    p.batch = a.batch; p.heads = a.heads; p.seq_q = a.seq_q; p.seq_k = a.seq_k;
    p.head_dim = a.head_dim; p.causal = a.causal;
    p.scale = a.scale > 0.0f ? a.scale : 1.0f / std::sqrt(static_cast<float>(a.head_dim));
    return p;
}

void account_attention(const vnpu_attention_f32_args_t &a, ExecStats &st)
{
    const uint64_t bh = static_cast<uint64_t>(a.batch) * a.heads;
    const uint64_t qn = bh * a.seq_q * a.head_dim, kn = bh * a.seq_k * a.head_dim;
    const uint64_t mn = a.mask ? bh * a.seq_q * a.seq_k : 0;
    st.bytes_read += (qn + 2 * kn + mn) * 4;
    st.bytes_written += qn * 4;
    st.flops += 4ull * a.batch * a.heads * a.seq_q * a.seq_k * a.head_dim;
}

void exec_attention(vnpu_stream_t *s, const vnpu_attention_f32_args_t &a, ExecStats &st)
{
    k::Attn p = attention_params(a);
    p.exact = s->device->reference_order;
    const uint64_t bh = static_cast<uint64_t>(a.batch) * a.heads;
    const uint64_t qn = bh * a.seq_q * a.head_dim, kn = bh * a.seq_k * a.head_dim;
    const uint64_t mn = a.mask ? bh * a.seq_q * a.seq_k : 0;
    Stager sg(s->hip, s);
    p.Q = sg.in(a.Q, qn * 4);
    p.K = sg.in(a.K, kn * 4);
    p.V = sg.in(a.V, kn * 4);
    p.mask = sg.in(a.mask, mn * 4);
    p.O = sg.out(a.O, qn * 4);
    float *ws = static_cast<float *>(s->ensure_workspace(k::attention_ws_bytes(p)));
    k::attention(s->hip, p, ws);
    VNPU_HIP(hipGetLastError());
    sg.finish();
    account_attention(a, st);
}

void exec_copy(vnpu_stream_t *s, const vnpu_copy_args_t &a, ExecStats &st)
{
    // execute_copy (scheduler.cpp:643-651): memmove semantics for host copies
    require(a.dst && a.src && a.bytes, "invalid copy arguments");
    const bool dd = is_device_pointer(a.dst), sd = is_device_pointer(a.src);
    if (!dd && !sd) {
        VNPU_HIP(hipStreamSynchronize(s->hip));
        std::memmove(a.dst, a.src, static_cast<size_t>(a.bytes));
    } else {
        VNPU_HIP(hipMemcpyAsync(a.dst, a.src, static_cast<size_t>(a.bytes), hipMemcpyDefault, s->hip));
        if (!dd || !sd) VNPU_HIP(hipStreamSynchronize(s->hip));
    }
    st.bytes_read += a.bytes;
    st.bytes_written += a.bytes;
    st.dma_bytes += a.bytes;
}

void exec_memset(vnpu_stream_t *s, const vnpu_memset_args_t &a, ExecStats &st)
{
    // execute_memset (scheduler.cpp:653-662)
    require(a.dst && a.bytes, "invalid memset arguments");
    if (is_device_pointer(a.dst)) {
        k::fill_u8(s->hip, a.dst, static_cast<uint8_t>(a.value & 0xffu), a.bytes);
    } else {
        VNPU_HIP(hipStreamSynchronize(s->hip));
        std::memset(a.dst, static_cast<int>(a.value & 0xffu), static_cast<size_t>(a.bytes));
    }
    VNPU_HIP(hipGetLastError());
    st.bytes_written += a.bytes;
    st.dma_bytes += a.bytes;
}

}  // namespace

void enqueue_attention_noalloc(vnpu_stream_t *s, const vnpu_attention_f32_args_t &a, ExecStats &st)
{
    k::Attn p = attention_params(a);
    p.exact = s->device->reference_order;
    // No staging: every tensor must already be device memory.
    require(is_device_pointer(a.Q) && is_device_pointer(a.K) && is_device_pointer(a.V) &&
                is_device_pointer(a.O) && (!a.mask || is_device_pointer(a.mask)),
            "attention without allocation needs device-resident Q, K, V, mask and O");
    p.Q = a.Q; p.K = a.K; p.V = a.V; p.mask = a.mask; p.O = a.O;
    const size_t need = k::attention_ws_bytes(p);
    if (need > k::kAttnScratchBytes) {
        debug_log("attention without allocation: this call needs %zu bytes of scratch, above the "
                  "%zu-byte device scratch", need, k::kAttnScratchBytes);
        throw ArgError("attention scratch requirement above the device scratch size");
    }
    float *ws = nullptr;
    if (need) {
        ws = k::attention_scratch(s->device->hip_device);
        if (!ws) throw HipError("attention scratch not set up on this device");
    }
    k::attention(s->hip, p, ws);
    VNPU_HIP(hipGetLastError());
    account_attention(a, st);
}

void execute_command(vnpu_device_t *dev, vnpu_stream_t *s, const vnpu_command_t &cmd,
                     uint32_t flags, ExecStats &st)
{
    switch (cmd.opcode) {
    case VNPU_OP_NOP:
    case VNPU_OP_BARRIER:
        return;
    case VNPU_OP_MATMUL_F32:
        exec_matmul_f32(dev, s, cmd.args.matmul_f32, flags, st);
        return;
    case VNPU_OP_MATMUL_I8:
        exec_matmul_i8(dev, s, cmd.args.matmul_i8, flags, st);
        return;
    case VNPU_OP_RMSNORM_F32:
        exec_rmsnorm(s, cmd.args.rmsnorm, st);
        return;
    case VNPU_OP_SOFTMAX_F32:
        exec_softmax(s, cmd.args.softmax, st);
        return;
    case VNPU_OP_ROPE_F32:
        exec_rope(dev, s, cmd.args.rope, st);
        return;
    case VNPU_OP_SWIGLU_F32:
    case VNPU_OP_GELU_F32:
    case VNPU_OP_ADD_F32:
    case VNPU_OP_MUL_F32:
        exec_elementwise(s, cmd, st);
        return;
    case VNPU_OP_ATTENTION_F32:
        exec_attention(s, cmd.args.attention, st);
        return;
    case VNPU_OP_QUANTIZE_I8:
        exec_quantize(dev, s, cmd.args.quantize_i8, st);
        return;
    case VNPU_OP_PACK_WEIGHTS_I8: {
        // execute_pack_weights (scheduler.cpp:664-677)
        const auto &a = cmd.args.pack_weights_i8;
        require(a.B && a.out && a.K && a.N, "invalid pack_weights arguments");
        VNPU_HIP(hipStreamSynchronize(s->hip));  // B may be produced earlier on this stream
        vnpu_packed_weights_t *w = pack_weights(dev, a.B, a.scales, a.K, a.N, a.ldb, a.trans_b);
        *a.out = w;
        st.bytes_read += static_cast<uint64_t>(a.K) * a.N * 2;
        st.bytes_written += w->frag_bytes;
        st.dma_bytes += static_cast<uint64_t>(a.K) * a.N * 2;
        return;
    }
    case VNPU_OP_MTP_HEAD_F32: {
        // execute_mtp_head (scheduler.cpp:610-641): a MATMUL_F32 with
        // M = gamma, K = hidden_dim, N = vocab, trans_b = trans_w.
        const auto &a = cmd.args.mtp_head;
        require(a.hidden && a.W && a.logits && a.gamma && a.hidden_dim && a.vocab,
                "invalid mtp_head arguments");
        vnpu_matmul_f32_args_t g{};
        g.A = a.hidden;
        g.B = a.W;
        g.bias = a.bias;
        g.C = a.logits;
        g.M = a.gamma;
        g.K = a.hidden_dim;
        g.N = a.vocab;
        g.trans_b = a.trans_w;
        g.alpha = 1.0f;
        g.unit = a.unit;
        exec_matmul_f32(dev, s, g, flags, st);
        return;
    }
    case VNPU_OP_COPY:
        exec_copy(s, cmd.args.copy, st);
        return;
    case VNPU_OP_MEMSET:
        exec_memset(s, cmd.args.memset, st);
        return;
    default:
        throw ArgError("invalid opcode");
    }
}

// ---------------------------------------------------------------------------
// Packed weights (reference scheduler.cpp:763-858)
// ---------------------------------------------------------------------------

vnpu_packed_weights_t *pack_weights(vnpu_device_t *dev, const int8_t *B, const float *scales,
                                    uint32_t K, uint32_t N, uint32_t ldb, uint32_t trans_b,
                                    const uint8_t *tile_mask, uint32_t mask_ld)
{
    const uint32_t ld = ldb ? ldb : (trans_b ? K : N);
    require(ld >= (trans_b ? K : N), "invalid pack ldb");
    const uint32_t mask_cols = (N + 63) / 64, mask_rows = (K + 63) / 64;
    const uint32_t mld = mask_ld ? mask_ld : mask_cols;
    require(!tile_mask || mld >= mask_cols, "invalid pack mask_ld");
    VNPU_HIP(hipSetDevice(dev->hip_device));
    std::unique_ptr<vnpu_packed_weights_t, void (*)(vnpu_packed_weights_t *)> w(
        new vnpu_packed_weights_t(), destroy_packed);
    w->device = dev;
    w->K = K;
    w->N = N;
    w->Kp = (K + 63) / 64 * 64;
    w->Np = (N + 15) / 16 * 16;
    const uint64_t blocks = static_cast<uint64_t>(w->Kp / 64) * (w->Np / 16);
    w->frag_bytes = blocks * 1024;
    VNPU_HIP(hipMalloc(&w->frag, w->frag_bytes));
    register_device_range(w->frag, w->frag_bytes);
    VNPU_HIP(hipMalloc(&w->scales_dev, static_cast<size_t>(w->Np) * 4));
    int32_t *sums_dev = nullptr;
    VNPU_HIP(hipMalloc(&sums_dev, static_cast<size_t>(N) * 4));
    std::unique_ptr<int32_t, hipError_t (*)(void *)> sums_guard(sums_dev, hipFree);

    hipStream_t st = nullptr;
    VNPU_HIP(hipStreamCreate(&st));
    std::unique_ptr<std::remove_pointer<hipStream_t>::type, hipError_t (*)(hipStream_t)> st_guard(
        st, hipStreamDestroy);
    const size_t b_bytes = trans_b ? span(N, K, ld, 1) : span(K, N, ld, 1);
    Stager sg(st);
    const int8_t *Bd = sg.in(B, b_bytes);
    const uint8_t *maskd =
        tile_mask ? sg.in(tile_mask, static_cast<size_t>(mask_rows - 1) * mld + mask_cols) : nullptr;
    k::pack_fragments(st, Bd, K, N, ld, trans_b, maskd, mld, w->frag, w->Kp, w->Np, sums_dev);
    VNPU_HIP(hipGetLastError());
    // Nonzero 64 x 64 tiles: per 64-column group, the k blocks to walk.
    const uint32_t groups = (w->Np / 16 + 3) / 4, kblocks = w->Kp / 64;
    VNPU_HIP(hipMalloc(&w->nz_list, static_cast<size_t>(groups) * kblocks * 4));
    VNPU_HIP(hipMalloc(&w->nz_count, static_cast<size_t>(groups) * 4));
    uint8_t *flag_dev = nullptr;
    VNPU_HIP(hipMalloc(&flag_dev, static_cast<size_t>(groups) * kblocks));
    std::unique_ptr<uint8_t, hipError_t (*)(void *)> flag_guard(flag_dev, hipFree);
    k::tile_lists(st, w->frag, w->Kp, w->Np, flag_dev, w->nz_list, w->nz_count);
    VNPU_HIP(hipGetLastError());
    std::vector<uint32_t> counts(groups);
    VNPU_HIP(hipMemcpyAsync(counts.data(), w->nz_count, static_cast<size_t>(groups) * 4, hipMemcpyDeviceToHost, st));

    // Scales: NULL keeps 1.0 (the reference does not derive them, F5 of its
    // scheduler.cpp:806-808).
    w->scales.assign(w->Np, 1.0f);
    if (scales) {
        if (is_device_pointer(scales))
            VNPU_HIP(hipMemcpyAsync(w->scales.data(), scales, static_cast<size_t>(N) * 4,
                                    hipMemcpyDeviceToHost, st));
        else
            std::memcpy(w->scales.data(), scales, static_cast<size_t>(N) * 4);
    }
    VNPU_HIP(hipStreamSynchronize(st));
    VNPU_HIP(hipMemcpy(w->scales_dev, w->scales.data(), static_cast<size_t>(w->Np) * 4,
                       hipMemcpyHostToDevice));
    w->column_sums.assign(w->Np, 0);
    VNPU_HIP(hipMemcpy(w->column_sums.data(), sums_dev, static_cast<size_t>(N) * 4,
                       hipMemcpyDeviceToHost));
    sg.finish();
    VNPU_HIP(hipStreamSynchronize(st));
    for (uint32_t c : counts) w->nz_tiles += c;
    dev->dma_bytes.fetch_add(static_cast<uint64_t>(K) * N * 2);
    return w.release();
}

void destroy_packed(vnpu_packed_weights_t *w)
{
    if (!w) return;
    if (w->frag) {
        unregister_device_range(w->frag);
        (void)hipFree(w->frag);
    }
    if (w->scales_dev) (void)hipFree(w->scales_dev);
    if (w->nz_list) (void)hipFree(w->nz_list);
    if (w->nz_count) (void)hipFree(w->nz_count);
    delete w;
}

void release_device_tables(vnpu_device_t *dev)
{
    {
        auto &c = inv_cache();
        std::lock_guard<std::mutex> lock(c.mutex);
        for (auto it = c.tables.begin(); it != c.tables.end();) {
            if (std::get<0>(it->first) == dev) {
                (void)hipFree(it->second);
                it = c.tables.erase(it);
            } else {
                ++it;
            }
        }
    }
    auto &c = rope_cs_cache();
    std::lock_guard<std::mutex> lock(c.mutex);
    for (auto it = c.tables.begin(); it != c.tables.end();) {
        if (std::get<0>(it->first) == dev) {
            (void)hipFree(it->second.table);
            for (float2 *r : it->second.retired) (void)hipFree(r);
            it = c.tables.erase(it);
        } else {
            ++it;
        }
    }
}

}  // namespace vnpu
