// cluster.cpp - the vnpu-node wire protocol, the node server and the cluster
// client, with the weights and the GEMM on the GPU.
//
// Wire format (reference src/cluster/protocol.h:45-119, kept byte for byte so
// either side interoperates with the reference's): a 32-byte native-endian
// header {magic "VPN1", version 1, op, request_id, payload_size, status (0 or
// -vnpu_status_t), flags, reserved} followed by the payload; ops HELLO, CAPS,
// PING, STORE_WEIGHTS (88-byte request + K*N floats), MATMUL_F32 (32-byte
// request + M*K floats; reply M*N floats), GET_STATS, SHUTDOWN; payloads up to
// 1 GiB; weight ids are FNV-1a 64 of "key:KxN".
//
// Node (reference src/cluster/node.cpp:81-270 semantics: per-connection
// HELLO/token gate, status replies, the same validation outcomes): stored
// weights live in HBM for the life of the node, in the layout they arrive in
// (trans_b is handed to MATMUL_F32 rather than transposed on the host); a
// MATMUL_F32 request's activations are received straight into pinned host
// memory, copied to HBM, multiplied on the node's stream and the result is
// copied back into pinned memory and sent.  One thread and one vnpu stream
// per connection.
//
// Cluster client (reference src/cluster/cluster.cpp:85-169, 240-546
// semantics): local workers are (device, stream) pairs and remote workers are
// node connections; GEMM rows are split by worker weight exactly as the
// reference splits them, and every worker runs its row range on its own
// thread.  Cached weights are uploaded once to HBM of every local device and
// stored once on every remote node.
#include "vnpu_internal.hpp"

#include <arpa/inet.h>
#include <netdb.h>
#include <netinet/in.h>
#include <netinet/tcp.h>
#include <sys/socket.h>
#include <sys/time.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <unordered_map>

namespace vnpu {
namespace wire {

constexpr uint32_t kMagic = 0x314e5056u;   // "VPN1"
constexpr uint32_t kVersion = 1u;
constexpr uint64_t kMaxPayload = 1ull << 30;

enum : uint32_t {
    OP_HELLO = 1,
    OP_CAPS = 2,
    OP_PING = 3,
    OP_STORE_WEIGHTS = 4,
    OP_MATMUL_F32 = 5,
    OP_GET_STATS = 6,
    OP_SHUTDOWN = 7,
};

#pragma pack(push, 1)
struct Header {
    uint32_t magic, version, op, request_id, payload_size, status, flags, reserved;
};
struct Hello {
    char token[64];
    char client_name[64];
    uint32_t abi_version;
    uint32_t flags;
};
struct Caps {
    uint32_t abi_version, num_threads, features_lo, features_hi;
    char backend[64];
    char node_name[64];
};
struct StoreWeights {
    uint64_t weight_id;
    uint32_t K, N, trans_b, reserved;
    char key[64];
};
struct MatmulF32 {
    uint64_t weight_id;
    uint32_t M, K, N, unit, flags, reserved;
};
struct Stats {
    uint64_t commands_completed, kernel_time_ns, flops, bytes_read, bytes_written, tiles_dispatched,
        tiles_culled;
};
#pragma pack(pop)
static_assert(sizeof(Header) == 32 && sizeof(Hello) == 136 && sizeof(Caps) == 144 &&
                  sizeof(StoreWeights) == 88 && sizeof(MatmulF32) == 32 && sizeof(Stats) == 56,
              "vnpu-node wire layout");

uint64_t fnv1a64(const std::string &s)
{
    uint64_t h = 1469598103934665603ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

uint64_t weight_id(const std::string &key, uint32_t K, uint32_t N)
{
    return fnv1a64(key + ":" + std::to_string(K) + "x" + std::to_string(N));
}

uint32_t encode_status(vnpu_status_t rc) { return rc == VNPU_OK ? 0u : static_cast<uint32_t>(-static_cast<int>(rc)); }

vnpu_status_t decode_status(uint32_t s)
{
    if (s == 0) return VNPU_OK;
    if (s < 1000) return static_cast<vnpu_status_t>(-static_cast<int>(s));
    return VNPU_ERR_PROTOCOL;
}

void set_timeouts(int fd, uint32_t ms)
{
    if (fd < 0 || !ms) return;
    timeval tv;
    tv.tv_sec = ms / 1000;
    tv.tv_usec = static_cast<long>(ms % 1000) * 1000;
    setsockopt(fd, SOL_SOCKET, SO_RCVTIMEO, &tv, sizeof(tv));
    setsockopt(fd, SOL_SOCKET, SO_SNDTIMEO, &tv, sizeof(tv));
}

void no_delay(int fd)
{
    int one = 1;
    setsockopt(fd, IPPROTO_TCP, TCP_NODELAY, &one, sizeof(one));
}

bool send_all(int fd, const void *data, size_t n)
{
    const char *p = static_cast<const char *>(data);
    while (n) {
        const ssize_t k = ::send(fd, p, std::min<size_t>(n, 1u << 20), MSG_NOSIGNAL);
        if (k > 0) {
            p += k;
            n -= static_cast<size_t>(k);
        } else if (k < 0 && errno == EINTR) {
            continue;
        } else {
            return false;
        }
    }
    return true;
}

bool recv_all(int fd, void *data, size_t n)
{
    char *p = static_cast<char *>(data);
    while (n) {
        const ssize_t k = ::recv(fd, p, std::min<size_t>(n, 1u << 20), 0);
        if (k > 0) {
            p += k;
            n -= static_cast<size_t>(k);
        } else if (k < 0 && errno == EINTR) {
            continue;
        } else {
            return false;   // closed, timed out or failed
        }
    }
    return true;
}

// Reads and discards n payload bytes (a rejected request's remainder).
bool drain(int fd, uint64_t n)
{
    char buf[16384];
    while (n) {
        const size_t k = static_cast<size_t>(std::min<uint64_t>(n, sizeof(buf)));
        if (!recv_all(fd, buf, k)) return false;
        n -= k;
    }
    return true;
}

vnpu_status_t send_message(int fd, uint32_t op, uint32_t id, const void *a, size_t na, const void *b = nullptr,
                           size_t nb = 0, uint32_t status = 0)
{
    if (fd < 0 || na + nb > kMaxPayload) return VNPU_ERR_NETWORK;
    Header h{kMagic, kVersion, op, id, static_cast<uint32_t>(na + nb), status, 0, 0};
    if (!send_all(fd, &h, sizeof(h))) return VNPU_ERR_NETWORK;
    if (na && !send_all(fd, a, na)) return VNPU_ERR_NETWORK;
    if (nb && !send_all(fd, b, nb)) return VNPU_ERR_NETWORK;
    return VNPU_OK;
}

vnpu_status_t recv_header(int fd, Header *h)
{
    if (fd < 0 || !recv_all(fd, h, sizeof(*h))) return VNPU_ERR_NETWORK;
    if (h->magic != kMagic || h->version != kVersion || h->payload_size > kMaxPayload) return VNPU_ERR_PROTOCOL;
    return VNPU_OK;
}

int connect_tcp(const char *host, uint16_t port, uint32_t timeout_ms)
{
    if (!host || !host[0]) host = "127.0.0.1";
    const std::string service = std::to_string(port);
    addrinfo hints{};
    hints.ai_family = AF_UNSPEC;
    hints.ai_socktype = SOCK_STREAM;
    hints.ai_protocol = IPPROTO_TCP;
    addrinfo *res = nullptr;
    if (getaddrinfo(host, service.c_str(), &hints, &res) != 0 || !res) return -1;
    int fd = -1;
    for (addrinfo *ai = res; ai; ai = ai->ai_next) {
        fd = ::socket(ai->ai_family, ai->ai_socktype, ai->ai_protocol);
        if (fd < 0) continue;
        set_timeouts(fd, timeout_ms);
        if (::connect(fd, ai->ai_addr, ai->ai_addrlen) == 0) break;
        ::close(fd);
        fd = -1;
    }
    freeaddrinfo(res);
    if (fd >= 0) no_delay(fd);
    return fd;
}

int listen_tcp(const char *bind_address, uint16_t port)
{
    if (!bind_address || !bind_address[0]) bind_address = "0.0.0.0";
    const std::string service = std::to_string(port);
    addrinfo hints{};
    hints.ai_family = AF_INET;
    hints.ai_socktype = SOCK_STREAM;
    hints.ai_protocol = IPPROTO_TCP;
    hints.ai_flags = AI_PASSIVE;
    addrinfo *res = nullptr;
    if (getaddrinfo(bind_address, service.c_str(), &hints, &res) != 0 || !res) return -1;
    int fd = ::socket(res->ai_family, res->ai_socktype, res->ai_protocol);
    if (fd >= 0) {
        int one = 1;
        setsockopt(fd, SOL_SOCKET, SO_REUSEADDR, &one, sizeof(one));
        if (::bind(fd, res->ai_addr, res->ai_addrlen) != 0 || ::listen(fd, 64) != 0) {
            ::close(fd);
            fd = -1;
        }
    }
    freeaddrinfo(res);
    return fd;
}

// True when a x b elements fit a payload (reference node.cpp:72-77).
bool shape_ok(uint64_t a, uint64_t b)
{
    if (!a || !b || a > std::numeric_limits<uint64_t>::max() / b) return false;
    return a * b <= kMaxPayload / sizeof(float);
}

}  // namespace wire

namespace {

uint64_t now_ns()
{
    return static_cast<uint64_t>(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
            .count());
}

// Pinned host memory that grows on demand (hipHostMalloc'd, page-locked, so
// the copies to and from HBM run at full PCIe rate).
struct Pinned {
    void *p = nullptr;
    size_t n = 0;
    void *get(size_t bytes)
    {
        if (bytes <= n) return p;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        n = 0;
        VNPU_HIP(hipHostMalloc(&p, bytes, hipHostMallocDefault));
        n = bytes;
        return p;
    }
    ~Pinned()
    {
        if (p) (void)hipHostFree(p);
    }
};

// HBM that grows on demand.
struct DevBuf {
    void *p = nullptr;
    size_t n = 0;
    int device = -1;
    void *get(int dev, size_t bytes)
    {
        if (bytes <= n) return p;
        if (p) {
            (void)hipSetDevice(device);
            (void)hipFree(p);
        }
        p = nullptr;
        n = 0;
        VNPU_HIP(hipSetDevice(dev));
        VNPU_HIP(hipMalloc(&p, bytes));
        device = dev;
        n = bytes;
        return p;
    }
    ~DevBuf()
    {
        if (p) {
            (void)hipSetDevice(device);
            (void)hipFree(p);
        }
    }
};

// -------------------------------------------------------------------------
// Node server
// -------------------------------------------------------------------------
// Freed by whoever drops the last reference: the weight map when a SET_WEIGHTS
// replaces it, or a MATMUL_F32 that still held it (it releases it only after
// its stream synchronized, so no kernel reads freed memory).
struct NodeWeights {
    void *dev = nullptr;       // HBM, as received: K x N, or N x K when trans_b
    int hip_device = 0;
    uint32_t K = 0, N = 0, trans_b = 0;
    NodeWeights() = default;
    NodeWeights(const NodeWeights &) = delete;
    NodeWeights &operator=(const NodeWeights &) = delete;
    ~NodeWeights()
    {
        if (dev) {
            (void)hipSetDevice(hip_device);
            (void)hipFree(dev);
        }
    }
};

struct NodeState {
    vnpu_device_t *device = nullptr;
    std::mutex weights_mutex;
    std::unordered_map<uint64_t, std::shared_ptr<NodeWeights>> weights;
    std::atomic<uint64_t> requests{0}, errors{0};
    std::string node_name;
};

std::atomic<bool> g_node_stop{false};
std::mutex g_server_mutex;
std::vector<int> g_listen_fds, g_client_fds;

void track(std::vector<int> &v, int fd, bool add)
{
    std::lock_guard<std::mutex> lock(g_server_mutex);
    if (add) v.push_back(fd);
    else v.erase(std::remove(v.begin(), v.end(), fd), v.end());
}

vnpu_status_t reply_status(int fd, uint32_t op, uint32_t id, vnpu_status_t rc)
{
    return wire::send_message(fd, op, id, nullptr, 0, nullptr, 0, wire::encode_status(rc));
}

void serve_client(int fd, std::shared_ptr<NodeState> st, std::string token)
{
    vnpu_stream_t *stream = nullptr;
    if (vnpu_stream_create(st->device, 0, &stream) != VNPU_OK) {
        track(g_client_fds, fd, false);
        ::close(fd);
        return;
    }
    const int dev = st->device->hip_device;
    Pinned host_a, host_c;
    DevBuf dev_a, dev_c;
    bool authenticated = false;
    try {
        for (;;) {
            wire::Header h{};
            if (wire::recv_header(fd, &h) != VNPU_OK) break;
            st->requests.fetch_add(1);
            const uint64_t size = h.payload_size;
            if (h.op == wire::OP_HELLO) {
                wire::Hello hello{};
                if (size < sizeof(hello)) {
                    wire::drain(fd, size);
                    reply_status(fd, h.op, h.request_id, VNPU_ERR_PROTOCOL);
                    break;
                }
                if (!wire::recv_all(fd, &hello, sizeof(hello)) || !wire::drain(fd, size - sizeof(hello))) break;
                hello.token[sizeof(hello.token) - 1] = '\0';
                if (!token.empty() && token != hello.token) {
                    reply_status(fd, h.op, h.request_id, VNPU_ERR_AUTH);
                    st->errors.fetch_add(1);
                    break;
                }
                authenticated = true;
                reply_status(fd, h.op, h.request_id, VNPU_OK);
                continue;
            }
            if (!authenticated) {
                wire::drain(fd, size);
                reply_status(fd, h.op, h.request_id, VNPU_ERR_AUTH);
                break;
            }
            switch (h.op) {
            case wire::OP_PING:
                if (!wire::drain(fd, size)) goto done;
                reply_status(fd, h.op, h.request_id, VNPU_OK);
                break;
            case wire::OP_CAPS: {
                if (!wire::drain(fd, size)) goto done;
                vnpu_device_info_t info{};
                vnpu_device_get_info(st->device, &info);
                wire::Caps caps{};
                caps.abi_version = VNPU_ABI_VERSION;
                caps.num_threads = info.num_threads;
                caps.features_lo = static_cast<uint32_t>(info.features);
                caps.features_hi = static_cast<uint32_t>(info.features >> 32);
                std::snprintf(caps.backend, sizeof(caps.backend), "%s", info.backend);
                std::snprintf(caps.node_name, sizeof(caps.node_name), "%s", st->node_name.c_str());
                wire::send_message(fd, h.op, h.request_id, &caps, sizeof(caps));
                break;
            }
            case wire::OP_STORE_WEIGHTS: {
                wire::StoreWeights req{};
                if (size < sizeof(req)) {
                    if (!wire::drain(fd, size)) goto done;
                    reply_status(fd, h.op, h.request_id, VNPU_ERR_PROTOCOL);
                    st->errors.fetch_add(1);
                    break;
                }
                if (!wire::recv_all(fd, &req, sizeof(req))) goto done;
                const uint64_t rest = size - sizeof(req);
                if (!wire::shape_ok(req.K, req.N)) {
                    if (!wire::drain(fd, rest)) goto done;
                    reply_status(fd, h.op, h.request_id, VNPU_ERR_INVALID_ARGUMENT);
                    break;
                }
                const uint64_t bytes = static_cast<uint64_t>(req.K) * req.N * sizeof(float);
                if (rest < bytes) {
                    if (!wire::drain(fd, rest)) goto done;
                    reply_status(fd, h.op, h.request_id, VNPU_ERR_PROTOCOL);
                    break;
                }
                void *pin = host_a.get(bytes);
                if (!wire::recv_all(fd, pin, bytes) || !wire::drain(fd, rest - bytes)) goto done;
                auto w = std::make_shared<NodeWeights>();
                w->K = req.K;
                w->N = req.N;
                w->trans_b = req.trans_b ? 1 : 0;
                w->hip_device = dev;
                VNPU_HIP(hipSetDevice(dev));
                VNPU_HIP(hipMalloc(&w->dev, bytes));
                VNPU_HIP(hipMemcpyAsync(w->dev, pin, bytes, hipMemcpyHostToDevice, stream->hip));
                VNPU_HIP(hipStreamSynchronize(stream->hip));
                std::shared_ptr<NodeWeights> old;   // freed below unless a MATMUL_F32 still holds it
                {
                    std::lock_guard<std::mutex> lock(st->weights_mutex);
                    auto &slot = st->weights[req.weight_id];
                    old.swap(slot);
                    slot = w;
                }
                old.reset();
                reply_status(fd, h.op, h.request_id, VNPU_OK);
                break;
            }
            case wire::OP_MATMUL_F32: {
                wire::MatmulF32 req{};
                if (size < sizeof(req)) {
                    if (!wire::drain(fd, size)) goto done;
                    reply_status(fd, h.op, h.request_id, VNPU_ERR_PROTOCOL);
                    break;
                }
                if (!wire::recv_all(fd, &req, sizeof(req))) goto done;
                const uint64_t rest = size - sizeof(req);
                if (!wire::shape_ok(req.M, req.K) || !wire::shape_ok(req.K, req.N) ||
                    !wire::shape_ok(req.M, req.N)) {
                    if (!wire::drain(fd, rest)) goto done;
                    reply_status(fd, h.op, h.request_id, VNPU_ERR_INVALID_ARGUMENT);
                    break;
                }
                const uint64_t a_bytes = static_cast<uint64_t>(req.M) * req.K * sizeof(float);
                if (rest < a_bytes) {
                    if (!wire::drain(fd, rest)) goto done;
                    reply_status(fd, h.op, h.request_id, VNPU_ERR_PROTOCOL);
                    break;
                }
                void *pin_a = host_a.get(a_bytes);
                if (!wire::recv_all(fd, pin_a, a_bytes) || !wire::drain(fd, rest - a_bytes)) goto done;
                std::shared_ptr<NodeWeights> w;
                {
                    std::lock_guard<std::mutex> lock(st->weights_mutex);
                    auto it = st->weights.find(req.weight_id);
                    if (it != st->weights.end()) w = it->second;
                }
                if (!w || w->K != req.K || w->N != req.N) {
                    reply_status(fd, h.op, h.request_id, VNPU_ERR_NOT_FOUND);
                    break;
                }
                const uint64_t c_bytes = static_cast<uint64_t>(req.M) * req.N * sizeof(float);
                float *da = static_cast<float *>(dev_a.get(dev, a_bytes));
                float *dc = static_cast<float *>(dev_c.get(dev, c_bytes));
                VNPU_HIP(hipMemcpyAsync(da, pin_a, a_bytes, hipMemcpyHostToDevice, stream->hip));
                vnpu_matmul_f32_args_t args{};
                args.A = da;
                args.B = static_cast<const float *>(w->dev);
                args.C = dc;
                args.M = req.M;
                args.K = req.K;
                args.N = req.N;
                args.trans_b = w->trans_b;
                args.alpha = 1.0f;
                args.beta = 0.0f;
                args.unit = req.unit;
                const vnpu_status_t rc = vnpu_matmul_f32(stream, &args);
                if (rc != VNPU_OK) {
                    reply_status(fd, h.op, h.request_id, rc);
                    st->errors.fetch_add(1);
                    break;
                }
                void *pin_c = host_c.get(c_bytes);
                VNPU_HIP(hipMemcpyAsync(pin_c, dc, c_bytes, hipMemcpyDeviceToHost, stream->hip));
                VNPU_HIP(hipStreamSynchronize(stream->hip));
                wire::send_message(fd, h.op, h.request_id, pin_c, c_bytes);
                break;
            }
            case wire::OP_GET_STATS: {
                if (!wire::drain(fd, size)) goto done;
                vnpu_device_status_t s{};
                vnpu_device_get_status(st->device, &s);
                wire::Stats out{s.commands_completed, s.kernel_time_ns, s.flops, s.bytes_read, s.bytes_written,
                                s.tiles_dispatched, s.tiles_culled};
                wire::send_message(fd, h.op, h.request_id, &out, sizeof(out));
                break;
            }
            case wire::OP_SHUTDOWN:
                if (!wire::drain(fd, size)) goto done;
                reply_status(fd, h.op, h.request_id, VNPU_OK);
                vnpu_node_stop();
                break;
            default:
                if (!wire::drain(fd, size)) goto done;
                reply_status(fd, h.op, h.request_id, VNPU_ERR_UNSUPPORTED);
                break;
            }
        }
    } catch (const std::exception &e) {
        debug_log("vnpu-node client: %s", e.what());
        st->errors.fetch_add(1);
    }
done:
    vnpu_stream_destroy(stream);
    track(g_client_fds, fd, false);
    ::close(fd);
}

}  // namespace
}  // namespace vnpu

// -------------------------------------------------------------------------
// Cluster client objects
// -------------------------------------------------------------------------
struct vnpu_remote_node {
    std::string host;
    uint16_t port = 0;
    std::string auth_token;
    uint32_t weight = 1, flags = 0;
    struct Conn {
        int fd = -1;
        bool healthy = false;
        std::mutex mutex;
    };
    std::vector<std::unique_ptr<Conn>> conns;
};

struct vnpu_weight_handle {
    std::string key;
    uint64_t id = 0;
    uint32_t K = 0, N = 0, trans_b = 0;
    std::vector<float> B;                        // canonical K x N (what a node is sent)
    std::map<vnpu_device_t *, float *> on_device;  // HBM copy per local device
};

struct vnpu_cluster {
    vnpu_cluster_config_t config{};
    std::string name, auth_token;
    struct Worker {
        bool local = true;
        vnpu_device_t *device = nullptr;
        vnpu_stream_t *stream = nullptr;
        vnpu_remote_node_t *remote = nullptr;
        vnpu_remote_node::Conn *conn = nullptr;
        uint32_t weight = 1;
    };
    std::vector<Worker> workers;
    std::vector<std::unique_ptr<vnpu_remote_node_t>> remotes;
    std::vector<std::unique_ptr<vnpu_weight_handle_t>> weights;
    std::atomic<uint64_t> local_jobs{0}, remote_jobs{0}, total_jobs{0}, bytes_sent{0}, bytes_received{0},
        failed_jobs{0}, local_time_ns{0}, remote_time_ns{0}, speedup_x1000{0};
};

namespace vnpu {
namespace {

std::atomic<uint32_t> g_request_id{1};

// One request and its reply on a connection (the connection's mutex held).
vnpu_status_t exchange(vnpu_cluster_t *cl, vnpu_remote_node::Conn *c, uint32_t op, const void *a, size_t na,
                       const void *b, size_t nb, std::vector<uint8_t> *reply, void *reply_into = nullptr,
                       size_t reply_bytes = 0)
{
    const uint32_t id = g_request_id.fetch_add(1);
    vnpu_status_t rc = wire::send_message(c->fd, op, id, a, na, b, nb);
    if (rc != VNPU_OK) {
        c->healthy = false;
        return rc;
    }
    cl->bytes_sent.fetch_add(sizeof(wire::Header) + na + nb);
    wire::Header h{};
    rc = wire::recv_header(c->fd, &h);
    if (rc != VNPU_OK) {
        c->healthy = false;
        return rc;
    }
    cl->bytes_received.fetch_add(sizeof(wire::Header) + h.payload_size);
    // A reply of the expected size lands straight in the caller's buffer.
    if (reply_into && h.payload_size == reply_bytes && h.op == op && h.request_id == id && h.status == 0) {
        if (!wire::recv_all(c->fd, reply_into, reply_bytes)) {
            c->healthy = false;
            return VNPU_ERR_NETWORK;
        }
    } else {
        std::vector<uint8_t> tmp(h.payload_size);
        if (h.payload_size && !wire::recv_all(c->fd, tmp.data(), tmp.size())) {
            c->healthy = false;
            return VNPU_ERR_NETWORK;
        }
        if (reply_into && h.op == op && h.request_id == id && h.status == 0) {
            // A longer reply carries the result in front; a shorter one is broken.
            if (tmp.size() < reply_bytes) return VNPU_ERR_PROTOCOL;
            std::memcpy(reply_into, tmp.data(), reply_bytes);
        }
        if (reply) reply->swap(tmp);
    }
    if (h.op != op || h.request_id != id) return VNPU_ERR_PROTOCOL;
    return wire::decode_status(h.status);
}

vnpu_status_t hello(vnpu_cluster_t *cl, vnpu_remote_node_t *r, vnpu_remote_node::Conn *c)
{
    wire::Hello m{};
    std::snprintf(m.token, sizeof(m.token), "%s", r->auth_token.c_str());
    std::snprintf(m.client_name, sizeof(m.client_name), "%s", cl->name.c_str());
    m.abi_version = VNPU_ABI_VERSION;
    m.flags = cl->config.flags;
    return exchange(cl, c, wire::OP_HELLO, &m, sizeof(m), nullptr, 0, nullptr);
}

vnpu_status_t connect(vnpu_cluster_t *cl, vnpu_remote_node_t *r, vnpu_remote_node::Conn *c)
{
    if (c->fd >= 0 && c->healthy) return VNPU_OK;
    if (c->fd >= 0) ::close(c->fd);
    c->fd = wire::connect_tcp(r->host.c_str(), r->port, cl->config.request_timeout_ms);
    if (c->fd < 0) {
        c->healthy = false;
        return VNPU_ERR_NETWORK;
    }
    const vnpu_status_t rc = hello(cl, r, c);
    c->healthy = rc == VNPU_OK;
    return rc;
}

vnpu_status_t store_remote(vnpu_cluster_t *cl, vnpu_remote_node_t *r, vnpu_weight_handle_t *w)
{
    auto *c = r->conns[0].get();
    std::lock_guard<std::mutex> lock(c->mutex);
    vnpu_status_t rc = connect(cl, r, c);
    if (rc != VNPU_OK) return rc;
    wire::StoreWeights req{};
    req.weight_id = w->id;
    req.K = w->K;
    req.N = w->N;
    req.trans_b = 0;
    std::snprintf(req.key, sizeof(req.key), "%s", w->key.c_str());
    const size_t bytes = w->B.size() * sizeof(float);
    if (sizeof(req) + bytes > wire::kMaxPayload) return VNPU_ERR_INVALID_ARGUMENT;
    return exchange(cl, c, wire::OP_STORE_WEIGHTS, &req, sizeof(req), w->B.data(), bytes, nullptr);
}

vnpu_status_t matmul_remote(vnpu_cluster_t *cl, vnpu_remote_node_t *r, vnpu_remote_node::Conn *c,
                            const vnpu_weight_handle_t *w, const float *A, float *C, uint32_t M, uint32_t K,
                            uint32_t N, uint32_t unit)
{
    std::lock_guard<std::mutex> lock(c->mutex);
    vnpu_status_t rc = connect(cl, r, c);
    if (rc != VNPU_OK) return rc;
    wire::MatmulF32 req{};
    req.weight_id = w->id;
    req.M = M;
    req.K = K;
    req.N = N;
    req.unit = unit;
    const size_t a_bytes = static_cast<size_t>(M) * K * sizeof(float);
    if (sizeof(req) + a_bytes > wire::kMaxPayload) return VNPU_ERR_INVALID_ARGUMENT;
    return exchange(cl, c, wire::OP_MATMUL_F32, &req, sizeof(req), A, a_bytes, nullptr, C,
                    static_cast<size_t>(M) * N * sizeof(float));
}

float *upload_weights(vnpu_device_t *d, const vnpu_weight_handle_t *w)
{
    float *p = nullptr;
    const size_t bytes = w->B.size() * sizeof(float);
    VNPU_HIP(hipSetDevice(d->hip_device));
    VNPU_HIP(hipMalloc(&p, bytes));
    if (hipMemcpy(p, w->B.data(), bytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(p);
        throw HipError("cluster weights upload failed");
    }
    register_device_range(p, bytes);
    return p;
}

void release_weights(vnpu_weight_handle_t *w)
{
    for (auto &kv : w->on_device) {
        unregister_device_range(kv.second);
        (void)hipSetDevice(kv.first->hip_device);
        (void)hipFree(kv.second);
    }
    w->on_device.clear();
}

}  // namespace
}  // namespace vnpu

using namespace vnpu;

VNPU_API vnpu_status_t VNPU_CALL vnpu_cluster_create(const vnpu_cluster_config_t *config,
                                                     vnpu_cluster_t **out_cluster)
{
    if (!out_cluster) return VNPU_ERR_INVALID_ARGUMENT;
    *out_cluster = nullptr;
    return guard([&]() -> vnpu_status_t {
        auto *cl = new vnpu_cluster_t();
        if (config) cl->config = *config;
        else vnpu_cluster_config_init(&cl->config);
        if (!cl->config.abi_version) cl->config.abi_version = VNPU_ABI_VERSION;
        if (!cl->config.num_streams) cl->config.num_streams = 1;
        if (!cl->config.request_timeout_ms) cl->config.request_timeout_ms = 30000;
        cl->name = cl->config.cluster_name ? cl->config.cluster_name : "vnpu-cluster";
        cl->auth_token = cl->config.auth_token ? cl->config.auth_token : "";
        *out_cluster = cl;
        return VNPU_OK;
    });
}

VNPU_API void VNPU_CALL vnpu_cluster_destroy(vnpu_cluster_t *cluster)
{
    if (!cluster) return;
    for (auto &w : cluster->workers)
        if (w.local && w.stream) vnpu_stream_destroy(w.stream);
    for (auto &r : cluster->remotes)
        for (auto &c : r->conns)
            if (c->fd >= 0) {
                ::close(c->fd);
                c->fd = -1;
            }
    for (auto &w : cluster->weights) release_weights(w.get());
    delete cluster;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_cluster_add_device(vnpu_cluster_t *cluster, vnpu_device_t *device,
                                                         uint32_t weight)
{
    if (!cluster || !device) return VNPU_ERR_INVALID_ARGUMENT;
    return guard([&]() -> vnpu_status_t {
        for (uint32_t i = 0; i < std::max<uint32_t>(1, cluster->config.num_streams); ++i) {
            vnpu_stream_t *s = nullptr;
            const vnpu_status_t rc = vnpu_stream_create(device, 0, &s);
            if (rc != VNPU_OK) return rc;
            vnpu_cluster::Worker w;
            w.local = true;
            w.device = device;
            w.stream = s;
            w.weight = weight ? weight : 1;
            cluster->workers.push_back(w);
        }
        // Weights cached before this device joined go to its HBM now.
        for (auto &h : cluster->weights)
            if (!h->on_device.count(device)) h->on_device[device] = upload_weights(device, h.get());
        return VNPU_OK;
    });
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_cluster_add_remote(vnpu_cluster_t *cluster,
                                                         const vnpu_remote_node_config_t *config,
                                                         vnpu_remote_node_t **out_node)
{
    if (!cluster || !config || !config->host || !config->port) return VNPU_ERR_INVALID_ARGUMENT;
    if (out_node) *out_node = nullptr;
    return guard([&]() -> vnpu_status_t {
        auto r = std::make_unique<vnpu_remote_node_t>();
        r->host = config->host;
        r->port = config->port;
        r->auth_token = config->auth_token ? config->auth_token : cluster->auth_token;
        r->weight = config->weight ? config->weight : 1;
        r->flags = config->flags;
        for (uint32_t i = 0; i < std::max<uint32_t>(1, cluster->config.num_streams); ++i) {
            auto c = std::make_unique<vnpu_remote_node::Conn>();
            if (connect(cluster, r.get(), c.get()) != VNPU_OK) {
                if (c->fd >= 0) ::close(c->fd);
                continue;
            }
            vnpu_cluster::Worker w;
            w.local = false;
            w.remote = r.get();
            w.conn = c.get();
            w.weight = r->weight;
            cluster->workers.push_back(w);
            r->conns.push_back(std::move(c));
        }
        if (r->conns.empty()) return VNPU_ERR_NETWORK;
        if (out_node) *out_node = r.get();
        cluster->remotes.push_back(std::move(r));
        return VNPU_OK;
    });
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_cluster_get_stats(const vnpu_cluster_t *cluster, vnpu_cluster_stats_t *stats)
{
    if (!cluster || !stats) return VNPU_ERR_INVALID_ARGUMENT;
    std::memset(stats, 0, sizeof(*stats));
    stats->local_jobs = cluster->local_jobs.load();
    stats->remote_jobs = cluster->remote_jobs.load();
    stats->total_jobs = cluster->total_jobs.load();
    stats->network_bytes_sent = cluster->bytes_sent.load();
    stats->network_bytes_received = cluster->bytes_received.load();
    stats->failed_jobs = cluster->failed_jobs.load();
    stats->local_time_ns = static_cast<double>(cluster->local_time_ns.load());
    stats->remote_time_ns = static_cast<double>(cluster->remote_time_ns.load());
    stats->speedup_estimate = static_cast<double>(cluster->speedup_x1000.load()) / 1000.0;
    return VNPU_OK;
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_cluster_cache_weights_f32(vnpu_cluster_t *cluster, const char *key,
                                                                const float *B, uint32_t K, uint32_t N,
                                                                uint32_t trans_b, vnpu_weight_handle_t **out_handle)
{
    if (!cluster || !B || !K || !N || !out_handle || trans_b > 1) return VNPU_ERR_INVALID_ARGUMENT;
    *out_handle = nullptr;
    return guard([&]() -> vnpu_status_t {
        auto h = std::make_unique<vnpu_weight_handle_t>();
        h->key = key && key[0] ? key : "weights-" + std::to_string(cluster->weights.size());
        h->id = wire::weight_id(h->key, K, N);
        h->K = K;
        h->N = N;
        h->trans_b = trans_b;
        h->B.resize(static_cast<size_t>(K) * N);
        if (trans_b) {
            for (uint32_t k = 0; k < K; ++k)
                for (uint32_t n = 0; n < N; ++n) h->B[static_cast<size_t>(k) * N + n] = B[static_cast<size_t>(n) * K + k];
        } else {
            std::memcpy(h->B.data(), B, h->B.size() * sizeof(float));
        }
        struct Undo {
            vnpu_weight_handle_t *w;
            ~Undo() { if (w) release_weights(w); }
        } undo{h.get()};
        for (auto &w : cluster->workers)
            if (w.local && !h->on_device.count(w.device)) h->on_device[w.device] = upload_weights(w.device, h.get());
        // One STORE_WEIGHTS per remote node, not per connection.
        for (auto &r : cluster->remotes) {
            const vnpu_status_t rc = store_remote(cluster, r.get(), h.get());
            if (rc != VNPU_OK) {
                cluster->failed_jobs.fetch_add(1);
                return rc;
            }
        }
        undo.w = nullptr;
        *out_handle = h.get();
        cluster->weights.push_back(std::move(h));
        return VNPU_OK;
    });
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_cluster_matmul_f32(vnpu_cluster_t *cluster, vnpu_weight_handle_t *weights,
                                                         const float *A, float *C, uint32_t M, uint32_t K,
                                                         uint32_t N, uint32_t unit)
{
    if (!cluster || !weights || !A || !C || !M || !K || !N) return VNPU_ERR_INVALID_ARGUMENT;
    if (weights->K != K || weights->N != N) return VNPU_ERR_INVALID_ARGUMENT;
    if (cluster->workers.empty()) return VNPU_ERR_DEVICE_ERROR;
    return guard([&]() -> vnpu_status_t {
        // Row split by worker weight (reference cluster.cpp:453-468).
        const size_t n = cluster->workers.size();
        uint64_t total = 0;
        for (const auto &w : cluster->workers) total += std::max<uint32_t>(1, w.weight);
        std::vector<uint32_t> start(n), rows(n);
        uint32_t cursor = 0;
        for (size_t i = 0; i < n; ++i) {
            uint32_t r = static_cast<uint32_t>(static_cast<uint64_t>(M) * std::max<uint32_t>(1, cluster->workers[i].weight) /
                                               total);
            if (i + 1 == n) r = M - cursor;
            if (cursor + r > M) r = M - cursor;
            start[i] = cursor;
            rows[i] = r;
            cursor += r;
        }
        std::vector<vnpu_status_t> result(n, VNPU_OK);
        std::vector<uint64_t> took(n, 0);
        std::vector<std::thread> threads;
        for (size_t i = 0; i < n; ++i) {
            if (!rows[i]) continue;
            threads.emplace_back([&, i]() {
                const vnpu_cluster::Worker &w = cluster->workers[i];
                const uint64_t t0 = now_ns();
                const float *a = A + static_cast<size_t>(start[i]) * K;
                float *c = C + static_cast<size_t>(start[i]) * N;
                vnpu_status_t rc;
                if (w.local) {
                    auto it = weights->on_device.find(w.device);
                    vnpu_matmul_f32_args_t args{};
                    args.A = a;
                    args.B = it != weights->on_device.end() ? it->second : weights->B.data();
                    args.C = c;
                    args.M = rows[i];
                    args.K = K;
                    args.N = N;
                    args.alpha = 1.0f;
                    args.unit = unit;
                    rc = vnpu_matmul_f32(w.stream, &args);
                    cluster->local_jobs.fetch_add(1);
                    cluster->local_time_ns.fetch_add(now_ns() - t0);
                } else {
                    rc = matmul_remote(cluster, w.remote, w.conn, weights, a, c, rows[i], K, N, unit);
                    cluster->remote_jobs.fetch_add(1);
                    cluster->remote_time_ns.fetch_add(now_ns() - t0);
                }
                took[i] = now_ns() - t0;
                result[i] = rc;
                if (rc != VNPU_OK) cluster->failed_jobs.fetch_add(1);
            });
        }
        for (auto &t : threads) t.join();
        cluster->total_jobs.fetch_add(1);
        uint64_t sum = 0, mx = 0;
        for (uint64_t t : took) {
            sum += t;
            mx = std::max(mx, t);
        }
        if (mx) cluster->speedup_x1000.store(static_cast<uint64_t>(1000.0 * sum / mx));
        for (vnpu_status_t rc : result)
            if (rc != VNPU_OK) return rc;
        return VNPU_OK;
    });
}

VNPU_API void VNPU_CALL vnpu_node_stop(void)
{
    g_node_stop.store(true);
    std::vector<int> fds;
    {
        std::lock_guard<std::mutex> lock(g_server_mutex);
        fds = g_listen_fds;
        fds.insert(fds.end(), g_client_fds.begin(), g_client_fds.end());
    }
    // shutdown() wakes accept()/recv(); each owner closes its own socket.
    for (int fd : fds) ::shutdown(fd, SHUT_RDWR);
}

VNPU_API vnpu_status_t VNPU_CALL vnpu_node_run(const vnpu_node_config_t *config)
{
    if (!config) return VNPU_ERR_INVALID_ARGUMENT;
    return guard([&]() -> vnpu_status_t {
        {
            std::lock_guard<std::mutex> lock(g_server_mutex);
            if (g_listen_fds.empty()) g_node_stop.store(false);
        }
        vnpu_config_t devcfg;
        vnpu_config_init(&devcfg);
        devcfg.num_threads = config->num_threads;
        devcfg.node_name = config->node_name ? config->node_name : "vnpu-node";
        vnpu_device_t *device = nullptr;
        vnpu_status_t rc = vnpu_device_create(&devcfg, &device);
        if (rc != VNPU_OK) return rc;
        auto st = std::make_shared<NodeState>();
        st->device = device;
        st->node_name = devcfg.node_name;
        const int lfd = wire::listen_tcp(config->bind_address, config->port);
        if (lfd < 0) {
            st.reset();
            vnpu_device_destroy(device);
            return VNPU_ERR_NETWORK;
        }
        track(g_listen_fds, lfd, true);
        vnpu_device_info_t info{};
        vnpu_device_get_info(device, &info);
        std::fprintf(stdout, "vnpu-node %s listening on %s:%u | %s | auth=%s\n", st->node_name.c_str(),
                     config->bind_address ? config->bind_address : "0.0.0.0", static_cast<unsigned>(config->port),
                     info.backend, config->auth_token && config->auth_token[0] ? "token" : "open");
        std::fflush(stdout);
        const std::string token = config->auth_token ? config->auth_token : "";
        std::vector<std::thread> clients;
        while (!g_node_stop.load()) {
            sockaddr_storage addr{};
            socklen_t len = sizeof(addr);
            const int cfd = ::accept(lfd, reinterpret_cast<sockaddr *>(&addr), &len);
            if (cfd < 0) {
                if (g_node_stop.load()) break;
                if (errno == EINTR || errno == ECONNABORTED) continue;
                break;
            }
            wire::set_timeouts(cfd, 30000);
            wire::no_delay(cfd);
            track(g_client_fds, cfd, true);
            if (g_node_stop.load()) ::shutdown(cfd, SHUT_RDWR);
            clients.emplace_back(serve_client, cfd, st, token);
        }
        track(g_listen_fds, lfd, false);
        ::close(lfd);
        for (auto &t : clients) t.join();
        st.reset();
        vnpu_device_destroy(device);
        return VNPU_OK;
    });
}
