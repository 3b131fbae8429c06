// api.cpp -- the C ABI of include/bmo_attn.h: ring allocation, argument
// checking, error reporting, readout/export, and the node-level drop-in for
// the reference's launch_decode_attention.
//
// Error behaviour mirrors src/bmo_api.cpp: nothing throws across the ABI
// (every entry point catches), int entry points return a status and record a
// message retrievable with bmo_kv_ring_last_error, and a failed create
// returns NULL after printing to stderr (src/bmo_api.cpp:196-205).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/bmo_attn.h"
#include "kernels.hpp"

struct bmo_kv_ring {
    bmo::RingGeom g{};
    int device = 0;
    uint8_t *mem = nullptr;  // every stripe (layout in ring_layout.hpp)
    uint8_t *stage = nullptr;  // prefill staging, grown on demand (guarded by stage_mu)
    int64_t stage_bytes = 0;
    std::mutex stage_mu;
    std::mutex mu;           // guards last_error
    std::string last_error;
};

namespace {

thread_local std::string t_create_error;

// Rings by base address, so the node-level launcher (which only receives the
// cache pointers, as the reference's does) can check a ring's geometry.
std::mutex g_registry_mu;
std::map<const void *, bmo_kv_ring_t *> g_registry;

// Copies the geometry of the ring whose allocation starts at base, under
// the registry lock (a concurrent bmo_kv_ring_free cannot leave a dangling
// pointer here).  False if base is not a ring's allocation.
bool registry_geometry(const void *base, bmo::RingGeom *g) {
    std::lock_guard<std::mutex> lk(g_registry_mu);
    auto it = g_registry.find(base);
    if (it == g_registry.end()) return false;
    *g = it->second->g;
    return true;
}

// Writes one line to stderr the first time a launcher without a status
// channel rejects its arguments (thread-safe).
void warn_once(std::atomic<bool> &warned, const char *fn, const char *why) {
    if (!warned.exchange(true)) std::fprintf(stderr, "[bmo_attn] %s: %s\n", fn, why);
}

constexpr float kLog2e = 1.4426950408889634f;

thread_local std::string t_last_fail;  // the calling thread's last ring failure

int fail(bmo_kv_ring_t *r, int code, const std::string &msg) {
    t_last_fail = msg;
    if (r) {
        std::lock_guard<std::mutex> lk(r->mu);
        r->last_error = msg;
    }
    return code;
}

void clear_error(bmo_kv_ring_t *r) {
    std::lock_guard<std::mutex> lk(r->mu);
    r->last_error.clear();
}

// Makes the ring's device current for the duration of a call.
struct DeviceGuard {
    int prev = -1;
    bool switched = false;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) {
            switched = hipSetDevice(dev) == hipSuccess;
        }
    }
    ~DeviceGuard() {
        if (switched) (void) hipSetDevice(prev);
    }
};

int hip_fail(bmo_kv_ring_t *r, hipError_t e, const char *what) {
    return fail(r, BMO_ATTN_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

int check_layer(bmo_kv_ring_t *r, int layer, const char *fn) {
    if (layer < 0 || layer >= r->g.n_layers)
        return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": layer out of range");
    return BMO_ATTN_OK;
}

float f16_to_f32_host(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t) h >> 10) & 0x1Fu;
    const uint32_t m = (uint32_t) h & 0x3FFu;
    uint32_t x;
    if (e == 0x1Fu) {
        x = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        float v = std::ldexp((float) m, -24);
        std::memcpy(&x, &v, 4);
        x |= sign;
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

// Copies the groups holding slots [t0, t0+n) of one stripe to host, packed
// back to back; *first receives the first group's index.
// (One 1-D copy per group rather than one strided hipMemcpy2D: under
// rocprofv3's kernel trace, hipMemcpy2D device-to-host returned wrong bytes
// for these strides on MI355X while 1-D copies of the same groups were
// exact.  These are the host-side readout paths, not the hot path.)
hipError_t fetch_groups(const bmo_kv_ring_t *r, const uint8_t *stripe, int t0, int n,
                        std::vector<uint8_t> &buf, int *first) {
    const int G = bmo::keys_per_group(r->g.head_dim);
    const int g0 = t0 / G, g1 = (t0 + n - 1) / G;
    *first = g0;
    buf.resize((size_t) (g1 - g0 + 1) * bmo::kGroupBytes);
    for (int g = g0; g <= g1; ++g) {
        const hipError_t e = hipMemcpy(buf.data() + (size_t) (g - g0) * bmo::kGroupBytes,
                                       stripe + (int64_t) g * r->g.group_stride, bmo::kGroupBytes,
                                       hipMemcpyDeviceToHost);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Writes packed groups back to their places in a stripe.
hipError_t store_groups(const bmo_kv_ring_t *r, uint8_t *stripe, const std::vector<uint8_t> &buf,
                        int first) {
    const size_t n = buf.size() / bmo::kGroupBytes;
    for (size_t i = 0; i < n; ++i) {
        const hipError_t e = hipMemcpy(stripe + (int64_t) (first + (int64_t) i) * r->g.group_stride,
                                       buf.data() + i * bmo::kGroupBytes, bmo::kGroupBytes,
                                       hipMemcpyHostToDevice);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// ggml block (scale bits, 16 code bytes) of K (which 0) or V (which 1) at
// slot, block blk, from packed groups starting at group `first`.
void read_block(const bmo::RingGeom &g, const std::vector<uint8_t> &buf, int first, int which,
                int slot, int blk, uint16_t *d, uint8_t *qs) {
    const bmo::RingGeom pg = bmo::packed_stripe_geom(g);
    const int64_t base = (int64_t) first * bmo::kGroupBytes;
    const uint8_t *codes = buf.data() + (which == 0 ? pg.kcode_offset(slot, blk)
                                                     : pg.vcode_offset(slot, blk)) - base;
    const uint8_t flip = which == 0 ? bmo::kKCodeZero : 0;
    for (int j = 0; j < 16; ++j) qs[j] = codes[j] ^ flip;
    std::memcpy(d, buf.data() + pg.scale_offset(slot, blk) - base + 2 * which, 2);
}

void write_block(const bmo::RingGeom &g, std::vector<uint8_t> &buf, int first, int which,
                 int slot, int blk, uint16_t d, const uint8_t *qs) {
    const bmo::RingGeom pg = bmo::packed_stripe_geom(g);
    const int64_t base = (int64_t) first * bmo::kGroupBytes;
    uint8_t *codes = buf.data() + (which == 0 ? pg.kcode_offset(slot, blk)
                                               : pg.vcode_offset(slot, blk)) - base;
    const uint8_t flip = which == 0 ? bmo::kKCodeZero : 0;
    for (int j = 0; j < 16; ++j) codes[j] = qs[j] ^ flip;
    std::memcpy(buf.data() + pg.scale_offset(slot, blk) - base + 2 * which, &d, 2);
}

}  // namespace

const char *bmo::ring_thread_last_error() { return t_last_fail.c_str(); }

extern "C" {

int64_t bmo_kv_ring_stripe_bytes(int head_dim, int n_ctx) {
    if ((head_dim != 64 && head_dim != 128) || n_ctx <= 0) return 0;
    return bmo::stripe_bytes_for(head_dim, n_ctx);
}

bmo_kv_ring_t *bmo_kv_ring_create(int n_layers, int n_sessions, int n_kv_heads, int head_dim,
                                  int n_ctx) {
    t_create_error.clear();
    auto reject = [](const std::string &m) -> bmo_kv_ring_t * {
        t_create_error = "bmo_kv_ring_create: " + m;
        std::fprintf(stderr, "[bmo_attn] %s\n", t_create_error.c_str());
        return nullptr;
    };
    if (n_layers <= 0 || n_sessions <= 0 || n_kv_heads <= 0)
        return reject("n_layers, n_sessions and n_kv_heads must be positive");
    if (head_dim != 64 && head_dim != 128) return reject("head_dim must be 64 or 128");
    if (n_ctx <= 0 || n_ctx > 65536) return reject("n_ctx must be in [1, 65536]");
    bmo_kv_ring_t *r = nullptr;
    auto release = [](bmo_kv_ring_t *x) {
        if (x->mem) (void) hipFree(x->mem);
        if (x->stage) (void) hipFree(x->stage);
        delete x;
    };
    try {
        r = new bmo_kv_ring();
        r->g = bmo::make_geom(n_layers, n_sessions, n_kv_heads, head_dim, n_ctx);
        if (hipGetDevice(&r->device) != hipSuccess) {
            delete r;
            return reject("no HIP device");
        }
        const int64_t total = r->g.total_bytes();
        hipError_t e = hipMalloc(&r->mem, (size_t) total);
        if (e != hipSuccess) {
            r->mem = nullptr;
            release(r);
            return reject(std::string("hipMalloc of ") + std::to_string(total) +
                          " bytes failed: " + hipGetErrorString(e));
        }
        bmo::launch_clear(r->mem, total, 0, 1, nullptr);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            release(r);
            return reject(std::string("allocation or initialisation failed: ") +
                          hipGetErrorString(e));
        }
        std::lock_guard<std::mutex> lk(g_registry_mu);
        g_registry[r->mem] = r;
        return r;
    } catch (const std::exception &ex) {
        if (r) release(r);
        return reject(ex.what());
    } catch (...) {
        if (r) release(r);
        return reject("unknown exception");
    }
}

void bmo_kv_ring_free(bmo_kv_ring_t *ring) {
    if (!ring) return;
    try {
        {
            std::lock_guard<std::mutex> lk(g_registry_mu);
            g_registry.erase(ring->mem);
        }
        DeviceGuard dg(ring->device);
        if (ring->mem) (void) hipFree(ring->mem);
        if (ring->stage) (void) hipFree(ring->stage);
    } catch (...) {
    }
    delete ring;
}

int bmo_kv_ring_geometry(const bmo_kv_ring_t *r, int *n_layers, int *n_sessions, int *n_kv_heads,
                         int *head_dim, int *n_ctx) {
    if (!r) return BMO_ATTN_ERR_NULL;
    if (n_layers) *n_layers = r->g.n_layers;
    if (n_sessions) *n_sessions = r->g.n_sessions;
    if (n_kv_heads) *n_kv_heads = r->g.n_kv_heads;
    if (head_dim) *head_dim = r->g.head_dim;
    if (n_ctx) *n_ctx = r->g.n_ctx;
    return BMO_ATTN_OK;
}

int64_t bmo_kv_ring_bytes(const bmo_kv_ring_t *r) { return r ? r->g.total_bytes() : 0; }

void *bmo_kv_ring_k_base(bmo_kv_ring_t *r) { return r ? r->mem : nullptr; }
void *bmo_kv_ring_v_base(bmo_kv_ring_t *r) { return r ? r->mem + bmo::kVCodeOff : nullptr; }

const char *bmo_kv_ring_last_error(const bmo_kv_ring_t *r) {
    if (!r) return t_create_error.empty() ? nullptr : t_create_error.c_str();
    // a copy per thread: another thread's call on the ring may replace the
    // ring's message while the caller still reads this one
    thread_local std::string t_copy;
    auto *m = const_cast<bmo_kv_ring_t *>(r);
    {
        std::lock_guard<std::mutex> lk(m->mu);
        t_copy = m->last_error;
    }
    return t_copy.empty() ? nullptr : t_copy.c_str();
}

int bmo_kv_ring_reset(bmo_kv_ring_t *r, int session, void *stream) {
    if (!r) return BMO_ATTN_ERR_NULL;
    try {
        if (session < -1 || session >= r->g.n_sessions)
            return fail(r, BMO_ATTN_ERR_ARG, "bmo_kv_ring_reset: session out of range");
        DeviceGuard dg(r->device);
        const bmo::RingGeom &g = r->g;
        if (session == -1) {
            bmo::launch_clear(r->mem, g.total_bytes(), 0, 1, (hipStream_t) stream);
        } else {
            // group g of layer l holds the session's n_kv_heads groups side by
            // side; (layer, group) pairs are group_stride apart
            bmo::launch_clear(r->mem + g.stripe_offset(0, session, 0),
                              (int64_t) g.n_kv_heads * bmo::kGroupBytes, g.group_stride,
                              g.n_layers * g.n_groups, (hipStream_t) stream);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(r, e, "bmo_kv_ring_reset");
        clear_error(r);
        return BMO_ATTN_OK;
    } catch (...) {
        return fail(r, BMO_ATTN_ERR_INTERNAL, "bmo_kv_ring_reset: unknown exception");
    }
}

int bmo_kv_ring_append(bmo_kv_ring_t *r, int layer, int n_batch, const int *session_ids,
                       const int *pos, const float *k_new, const float *v_new, void *stream) {
    if (!r) return BMO_ATTN_ERR_NULL;
    try {
        if (!pos || !k_new || !v_new)
            return fail(r, BMO_ATTN_ERR_NULL, "bmo_kv_ring_append: null pointer argument");
        if (int rc = check_layer(r, layer, "bmo_kv_ring_append")) return rc;
        if (n_batch <= 0 || n_batch > r->g.n_sessions)
            return fail(r, BMO_ATTN_ERR_ARG, "bmo_kv_ring_append: n_batch must be in [1, n_sessions]");
        DeviceGuard dg(r->device);
        bmo::AppendParams p{};
        p.base = r->mem;
        p.g = r->g;
        p.layer = layer;
        p.n_rows = n_batch;
        p.session_ids = session_ids;
        p.pos = pos;
        p.k = k_new;
        p.v = v_new;
        bmo::launch_append(p, (hipStream_t) stream);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(r, e, "bmo_kv_ring_append");
        clear_error(r);
        return BMO_ATTN_OK;
    } catch (...) {
        return fail(r, BMO_ATTN_ERR_INTERNAL, "bmo_kv_ring_append: unknown exception");
    }
}

static int decode_common(bmo_kv_ring_t *r, const char *fn, bool fused, int layer, int n_batch,
                         const int *session_ids, const int *pos, int n_heads, const float *q,
                         const float *k_new, const float *v_new, float *out, float scale,
                         float rope_theta, void *stream) {
    if (!r) return BMO_ATTN_ERR_NULL;
    try {
        if (!pos || !q || !out || (fused && (!k_new || !v_new)))
            return fail(r, BMO_ATTN_ERR_NULL, std::string(fn) + ": null pointer argument");
        if (int rc = check_layer(r, layer, fn)) return rc;
        if (n_batch <= 0 || n_batch > r->g.n_sessions)
            return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": n_batch must be in [1, n_sessions]");
        if (n_heads <= 0 || n_heads % r->g.n_kv_heads != 0)
            return fail(r, BMO_ATTN_ERR_ARG,
                        std::string(fn) + ": n_heads must be a positive multiple of n_kv_heads");
        if ((int64_t) n_batch * n_heads > INT_MAX)
            return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": n_batch * n_heads exceeds INT_MAX");
        if (!(scale > 0.0f)) scale = 1.0f / std::sqrt((float) r->g.head_dim);
        if (!std::isfinite(scale))
            return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": scale must be finite");
        if (rope_theta != 0.0f && !(rope_theta > 0.0f && std::isfinite(rope_theta)))
            return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": rope_theta must be positive and finite");
        DeviceGuard dg(r->device);
        bmo::DecodeParams p{};
        p.rope = rope_theta != 0.0f;
        p.rope_r = p.rope ? std::pow((double) rope_theta, -2.0 / (double) r->g.head_dim) : 0.0;
        p.base = r->mem;
        p.g = r->g;
        p.layer = layer;
        p.n_batch = n_batch;
        p.n_heads = n_heads;
        p.n_kv = r->g.n_kv_heads;
        p.session_ids = session_ids;
        p.pos = pos;
        p.q = q;
        p.k_new = k_new;
        p.v_new = v_new;
        p.out = out;
        p.qscale = scale * kLog2e;
        if (!bmo::launch_decode(p, fused, (hipStream_t) stream))
            return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": unsupported head_dim");
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(r, e, fn);
        clear_error(r);
        return BMO_ATTN_OK;
    } catch (...) {
        return fail(r, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

int bmo_kv_ring_decode(bmo_kv_ring_t *r, int layer, int n_batch, const int *session_ids,
                       const int *pos, int n_heads, const float *q, float *out, float scale,
                       void *stream) {
    return decode_common(r, "bmo_kv_ring_decode", false, layer, n_batch, session_ids, pos, n_heads,
                         q, nullptr, nullptr, out, scale, 0.0f, stream);
}

int bmo_kv_ring_append_decode(bmo_kv_ring_t *r, int layer, int n_batch, const int *session_ids,
                              const int *pos, int n_heads, const float *q, const float *k_new,
                              const float *v_new, float *out, float scale, void *stream) {
    return decode_common(r, "bmo_kv_ring_append_decode", true, layer, n_batch, session_ids, pos,
                         n_heads, q, k_new, v_new, out, scale, 0.0f, stream);
}

int bmo_kv_ring_append_decode_rope(bmo_kv_ring_t *r, int layer, int n_batch,
                                   const int *session_ids, const int *pos, int n_heads,
                                   const float *q, const float *k_new, const float *v_new,
                                   float *out, float scale, float rope_theta, void *stream) {
    if (r && !(rope_theta > 0.0f))
        return fail(r, BMO_ATTN_ERR_ARG, "bmo_kv_ring_append_decode_rope: rope_theta must be positive");
    return decode_common(r, "bmo_kv_ring_append_decode_rope", true, layer, n_batch, session_ids,
                         pos, n_heads, q, k_new, v_new, out, scale, rope_theta, stream);
}

int bmo_kv_ring_write(bmo_kv_ring_t *r, int layer, int session, int64_t pos0, int n_tok,
                      const float *k, const float *v, void *stream) {
    if (!r) return BMO_ATTN_ERR_NULL;
    try {
        if (!k || !v) return fail(r, BMO_ATTN_ERR_NULL, "bmo_kv_ring_write: null pointer argument");
        if (int rc = check_layer(r, layer, "bmo_kv_ring_write")) return rc;
        if (session < 0 || session >= r->g.n_sessions)
            return fail(r, BMO_ATTN_ERR_ARG, "bmo_kv_ring_write: session out of range");
        if (pos0 < 0) return fail(r, BMO_ATTN_ERR_ARG, "bmo_kv_ring_write: pos0 must be >= 0");
        if (n_tok <= 0 || n_tok > r->g.n_ctx)
            return fail(r, BMO_ATTN_ERR_ARG, "bmo_kv_ring_write: n_tok must be in [1, n_ctx]");
        DeviceGuard dg(r->device);
        bmo::AppendParams p{};
        p.base = r->mem;
        p.g = r->g;
        p.layer = layer;
        p.n_rows = n_tok;
        p.session = session;
        p.pos0 = pos0;
        p.k = k;
        p.v = v;
        bmo::launch_append(p, (hipStream_t) stream);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(r, e, "bmo_kv_ring_write");
        clear_error(r);
        return BMO_ATTN_OK;
    } catch (...) {
        return fail(r, BMO_ATTN_ERR_INTERNAL, "bmo_kv_ring_write: unknown exception");
    }
}

}  // extern "C"

namespace {

// Staging of bmo_kv_ring_prefill_noalloc: a fixed array in each device's
// global memory (the library holds it until the process ends), shared by
// every such call on that device.  Host code uses the per-device address
// from hipGetSymbolAddress, never the array's name (which is a host-side
// stand-in).  Staged blocks are written by the stage kernel of the same call
// before anything reads them (padding slots are read only under a zero
// scale and a mask), so nothing needs clearing between calls.
constexpr int64_t kNoAllocScratchBytes = int64_t(32) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[kMaxDevices] = {};

// The scratch address on `device` (which must be current), looked up once
// per device; nullptr with *err set on failure.
uint8_t *scratch_on(int device, hipError_t *err) {
    *err = hipSuccess;
    if (device < 0 || device >= kMaxDevices) {
        *err = hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *ptr = nullptr;
        *err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (*err != hipSuccess) return nullptr;
        g_scratch_ptr[device] = static_cast<uint8_t *>(ptr);
    }
    return g_scratch_ptr[device];
}

int prefill_common(bmo_kv_ring_t *r, const char *fn, bool noalloc, int layer, int n_batch,
                   const int *session_ids, const int *pos0, int n_tok, int n_heads, const uint16_t *q,
                   const uint16_t *k, const uint16_t *v, float *out, float scale, void *stream) {
    if (!r) return BMO_ATTN_ERR_NULL;
    try {
        if (!pos0 || !q || !k || !v || !out)
            return fail(r, BMO_ATTN_ERR_NULL, std::string(fn) + ": null pointer argument");
        if (int rc = check_layer(r, layer, fn)) return rc;
        if (n_batch <= 0 || n_batch > r->g.n_sessions)
            return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": n_batch must be in [1, n_sessions]");
        if (n_tok <= 0 || n_tok > r->g.n_ctx)
            return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": n_tok must be in [1, n_ctx]");
        if (n_heads <= 0 || n_heads % r->g.n_kv_heads != 0)
            return fail(r, BMO_ATTN_ERR_ARG,
                        std::string(fn) + ": n_heads must be a positive multiple of n_kv_heads");
        if (!(scale > 0.0f)) scale = 1.0f / std::sqrt((float) r->g.head_dim);
        if (!std::isfinite(scale))
            return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": scale must be finite");
        if ((int64_t) n_batch * n_tok * r->g.n_kv_heads * (r->g.head_dim / 32) * 2 > INT32_MAX)
            return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": chunk too large (2^31 Q4_0 blocks)");
        if (r->g.group_stride > (int64_t) UINT32_MAX)
            return fail(r, BMO_ATTN_ERR_ARG,
                        std::string(fn) + ": n_sessions * n_kv_heads too large for prefill");
        DeviceGuard dg(r->device);
        bmo::PrefillParams p{};
        p.base = r->mem;
        p.g = r->g;
        p.layer = layer;
        p.n_batch = n_batch;
        p.n_heads = n_heads;
        p.n_kv = r->g.n_kv_heads;
        p.session_ids = session_ids;
        p.pos0 = pos0;
        p.n_tok = n_tok;
        p.q = q;
        p.k = k;
        p.v = v;
        p.out = out;
        p.qscale = scale * kLog2e;
        p.sg = bmo::make_geom(1, n_batch, r->g.n_kv_heads, r->g.head_dim, n_tok);
        const int64_t need = bmo::prefill_is_direct(p) ? 0 : p.sg.total_bytes();
        std::unique_lock<std::mutex> stage_lock(r->stage_mu, std::defer_lock);
        if (noalloc) {
            if (need > kNoAllocScratchBytes)
                return fail(r, BMO_ATTN_ERR_ARG,
                            std::string(fn) + ": the staged chunk needs " + std::to_string(need) +
                                " bytes (n_batch * n_kv_heads * ceil(n_tok / (2048 / head_dim)) * "
                                "2304), more than the " + std::to_string(kNoAllocScratchBytes) +
                                "-byte scratch");
            if (need > 0) {
                hipError_t e;
                p.stage = scratch_on(r->device, &e);
                if (!p.stage) return hip_fail(r, e, (std::string(fn) + ": scratch address").c_str());
            }
        } else {
            // Staged calls on one ring share its staging buffer: they must be
            // ordered on one stream (the lock only guards the buffer's growth).
            stage_lock.lock();
            if (need > r->stage_bytes) {
                // grow-only staging; the previous one may still be read by queued work
                hipError_t e = hipStreamSynchronize((hipStream_t) stream);
                if (e == hipSuccess && r->stage) e = hipFree(r->stage);
                r->stage = nullptr;
                r->stage_bytes = 0;
                if (e == hipSuccess) e = hipMalloc(&r->stage, (size_t) need);
                if (e != hipSuccess) {
                    r->stage = nullptr;
                    return hip_fail(r, e, "bmo_kv_ring_prefill: staging allocation");
                }
                r->stage_bytes = need;
            }
            p.stage = r->stage;
        }
        if (!bmo::launch_prefill(p, (hipStream_t) stream))
            return fail(r, BMO_ATTN_ERR_ARG, std::string(fn) + ": unsupported head_dim");
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(r, e, fn);
        clear_error(r);
        return BMO_ATTN_OK;
    } catch (...) {
        return fail(r, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

}  // namespace

extern "C" {

int bmo_kv_ring_prefill(bmo_kv_ring_t *r, int layer, int n_batch, const int *session_ids,
                        const int *pos0, int n_tok, int n_heads, const uint16_t *q,
                        const uint16_t *k, const uint16_t *v, float *out, float scale,
                        void *stream) {
    return prefill_common(r, "bmo_kv_ring_prefill", false, layer, n_batch, session_ids, pos0, n_tok,
                          n_heads, q, k, v, out, scale, stream);
}

int bmo_kv_ring_prefill_noalloc(bmo_kv_ring_t *r, int layer, int n_batch, const int *session_ids,
                                const int *pos0, int n_tok, int n_heads, const uint16_t *q,
                                const uint16_t *k, const uint16_t *v, float *out, float scale,
                                void *stream) {
    return prefill_common(r, "bmo_kv_ring_prefill_noalloc", true, layer, n_batch, session_ids, pos0,
                          n_tok, n_heads, q, k, v, out, scale, stream);
}

int bmo_kv_ring_copy_k_f32(bmo_kv_ring_t *r, int layer, int session, int t_start, int n_positions,
                           float *out, int max_floats) {
    if (!r || !out || n_positions <= 0 || max_floats <= 0) return BMO_ATTN_READ_ERR_NULL;
    try {
        const bmo::RingGeom &g = r->g;
        if (session < 0 || session >= g.n_sessions) return BMO_ATTN_READ_ERR_NULL;
        if (layer < 0 || layer >= g.n_layers) return BMO_ATTN_READ_ERR_RANGE;
        if (t_start < 0 || (int64_t) t_start + n_positions > g.n_ctx) return BMO_ATTN_READ_ERR_RANGE;
        const int64_t need = (int64_t) n_positions * g.n_kv_heads * g.head_dim;
        if (need > (int64_t) max_floats) return BMO_ATTN_READ_ERR_SMALL;
        DeviceGuard dg(r->device);
        if (hipDeviceSynchronize() != hipSuccess) return BMO_ATTN_READ_ERR_NULL;
        const int D = g.head_dim;
        const int nblk = D / bmo::kQK;
        std::vector<uint8_t> buf;
        int first = 0;
        for (int h = 0; h < g.n_kv_heads; ++h) {
            if (fetch_groups(r, r->mem + g.stripe_offset(layer, session, h), t_start, n_positions,
                             buf, &first) != hipSuccess)
                return BMO_ATTN_READ_ERR_NULL;
            for (int ti = 0; ti < n_positions; ++ti) {
                float *o = out + ((int64_t) ti * g.n_kv_heads + h) * D;
                for (int b = 0; b < nblk; ++b) {
                    uint16_t d16;
                    uint8_t qs[16];
                    read_block(g, buf, first, 0, t_start + ti, b, &d16, qs);
                    const float d = f16_to_f32_host(d16);
                    for (int j = 0; j < 16; ++j) {
                        o[b * 32 + j] = (float) ((int) (qs[j] & 0x0F) - 8) * d;
                        o[b * 32 + j + 16] = (float) ((int) (qs[j] >> 4) - 8) * d;
                    }
                }
            }
        }
        return (int) need;
    } catch (...) {
        return BMO_ATTN_READ_ERR_NULL;
    }
}

int64_t bmo_kv_ring_export_q4_0(bmo_kv_ring_t *r, int layer, int session, int which, int t_start,
                                int n_positions, void *out, int64_t max_bytes) {
    if (!r || !out || n_positions <= 0 || max_bytes <= 0) return BMO_ATTN_READ_ERR_NULL;
    try {
        const bmo::RingGeom &g = r->g;
        if (session < 0 || session >= g.n_sessions || (which != 0 && which != 1))
            return BMO_ATTN_READ_ERR_NULL;
        if (layer < 0 || layer >= g.n_layers) return BMO_ATTN_READ_ERR_RANGE;
        if (t_start < 0 || (int64_t) t_start + n_positions > g.n_ctx) return BMO_ATTN_READ_ERR_RANGE;
        const int nblk = g.head_dim / bmo::kQK;
        const int64_t need = (int64_t) n_positions * g.n_kv_heads * nblk * 18;
        if (need > max_bytes) return BMO_ATTN_READ_ERR_SMALL;
        DeviceGuard dg(r->device);
        if (hipDeviceSynchronize() != hipSuccess) return BMO_ATTN_READ_ERR_NULL;
        uint8_t *dst = static_cast<uint8_t *>(out);
        std::vector<uint8_t> buf;
        int first = 0;
        for (int h = 0; h < g.n_kv_heads; ++h) {
            if (fetch_groups(r, r->mem + g.stripe_offset(layer, session, h), t_start, n_positions,
                             buf, &first) != hipSuccess)
                return BMO_ATTN_READ_ERR_NULL;
            for (int ti = 0; ti < n_positions; ++ti)
                for (int b = 0; b < nblk; ++b) {
                    uint8_t *blkp = dst + (((int64_t) ti * g.n_kv_heads + h) * nblk + b) * 18;
                    uint16_t d16;
                    read_block(g, buf, first, which, t_start + ti, b, &d16, blkp + 2);
                    std::memcpy(blkp, &d16, 2);
                }
        }
        return need;
    } catch (...) {
        return BMO_ATTN_READ_ERR_NULL;
    }
}

int64_t bmo_kv_ring_import_q4_0(bmo_kv_ring_t *r, int layer, int session, int which, int t_start,
                                int n_positions, const void *in, int64_t n_bytes) {
    if (!r || !in || n_positions <= 0 || n_bytes <= 0) return BMO_ATTN_READ_ERR_NULL;
    try {
        const bmo::RingGeom &g = r->g;
        if (session < 0 || session >= g.n_sessions || (which != 0 && which != 1))
            return BMO_ATTN_READ_ERR_NULL;
        if (layer < 0 || layer >= g.n_layers) return BMO_ATTN_READ_ERR_RANGE;
        if (t_start < 0 || (int64_t) t_start + n_positions > g.n_ctx) return BMO_ATTN_READ_ERR_RANGE;
        const int nblk = g.head_dim / bmo::kQK;
        const int64_t need = (int64_t) n_positions * g.n_kv_heads * nblk * 18;
        if (n_bytes < need) return BMO_ATTN_READ_ERR_SMALL;
        DeviceGuard dg(r->device);
        if (hipDeviceSynchronize() != hipSuccess) return BMO_ATTN_READ_ERR_NULL;
        const uint8_t *src = static_cast<const uint8_t *>(in);
        std::vector<uint8_t> buf;
        int first = 0;
        for (int h = 0; h < g.n_kv_heads; ++h) {
            uint8_t *stripe = r->mem + g.stripe_offset(layer, session, h);
            // read-modify-write: a group also holds other slots and the other
            // half of each scale dword
            if (fetch_groups(r, stripe, t_start, n_positions, buf, &first) != hipSuccess)
                return BMO_ATTN_READ_ERR_NULL;
            for (int ti = 0; ti < n_positions; ++ti)
                for (int b = 0; b < nblk; ++b) {
                    const uint8_t *blkp = src + (((int64_t) ti * g.n_kv_heads + h) * nblk + b) * 18;
                    uint16_t d16;
                    std::memcpy(&d16, blkp, 2);
                    write_block(g, buf, first, which, t_start + ti, b, d16, blkp + 2);
                }
            if (store_groups(r, stripe, buf, first) != hipSuccess) return BMO_ATTN_READ_ERR_NULL;
        }
        return need;
    } catch (...) {
        return BMO_ATTN_READ_ERR_NULL;
    }
}

int bmo_positions_advance(int *pos_dev, int n, int delta, void *stream) {
    if (!pos_dev) return BMO_ATTN_ERR_NULL;
    if (n <= 0) return BMO_ATTN_ERR_ARG;
    bmo::launch_advance(pos_dev, n, delta, (hipStream_t) stream);
    return hipGetLastError() == hipSuccess ? BMO_ATTN_OK : BMO_ATTN_ERR_HIP;
}

int bmo_launch_gemv_q4_0_q8_1(const void *W_dev, const float *x_dev, float *y_dev, int rows,
                              int cols, void *q8_scratch, void *stream) {
    // Same arguments as src/bmo_cuda_kernels.cu:685-711 (which returns
    // nothing); rejected arguments launch nothing, are reported once on
    // stderr and return an error code.
    static std::atomic<bool> warned{false};
    auto reject = [](int code, const char *why) {
        warn_once(warned, "bmo_launch_gemv_q4_0_q8_1", why);
        return code;
    };
    try {
        if (!W_dev || !x_dev || !y_dev) return reject(BMO_ATTN_ERR_NULL, "null pointer argument");
        if (rows <= 0 || cols <= 0 || cols % 64 != 0)
            return reject(BMO_ATTN_ERR_ARG, "rows must be positive and cols a positive multiple of 64");
        if (bmo::gemv_lds_bytes(cols) > 64 * 1024)
            return reject(BMO_ATTN_ERR_ARG, "cols too large (at most 52428)");
        if ((reinterpret_cast<uintptr_t>(W_dev) & 3) || (reinterpret_cast<uintptr_t>(x_dev) & 15) ||
            (reinterpret_cast<uintptr_t>(q8_scratch) & 3))
            return reject(BMO_ATTN_ERR_ARG, "W_dev and q8_scratch must be 4-byte, x_dev 16-byte aligned");
        bmo::GemvParams p{};
        p.w = static_cast<const uint8_t *>(W_dev);
        p.x = x_dev;
        p.y = y_dev;
        p.rows = rows;
        p.cols = cols;
        p.q8_out = static_cast<uint8_t *>(q8_scratch);
        bmo::launch_gemv(p, (hipStream_t) stream);
        if (hipGetLastError() != hipSuccess) return reject(BMO_ATTN_ERR_HIP, "launch failed");
        return BMO_ATTN_OK;
    } catch (...) {
        return reject(BMO_ATTN_ERR_INTERNAL, "unknown exception");
    }
}

void bmo_launch_decode_attention(const float *q_dev, const float *k_dev, const float *v_dev,
                                 void *k_cache_dev, void *v_cache_dev, float *out_dev, int head_dim,
                                 int n_heads, int n_kv_heads, int n_ctx, int n_past, int layer,
                                 void *stream, const int *pos_dev) {
    // Mirrors src/bmo_cuda_kernels.cu:850-884: no status is returned, so
    // rejected arguments launch nothing (as an invalid launch would) and are
    // reported on stderr once.
    static std::atomic<bool> warned{false};
    auto reject = [](const char *why) { warn_once(warned, "bmo_launch_decode_attention", why); };
    if (!q_dev || !k_dev || !v_dev || !k_cache_dev || !v_cache_dev || !out_dev ||
        (head_dim != 64 && head_dim != 128) || n_heads <= 0 || n_kv_heads <= 0 ||
        n_heads % n_kv_heads != 0 || n_ctx <= 0 || n_ctx > 65536 || layer < 0 ||
        (pos_dev == nullptr && n_past < 0))
        return reject("invalid arguments");
    // Both cache pointers address the one ring allocation.
    if (static_cast<uint8_t *>(v_cache_dev) != static_cast<uint8_t *>(k_cache_dev) + bmo::kVCodeOff)
        return reject("v_cache_dev must be bmo_kv_ring_v_base of the ring whose k_base is k_cache_dev");
    bmo::DecodeParams p{};
    // The reference cache has n_heads head slots per layer and one session.
    p.g = bmo::make_geom(layer + 1, 1, n_heads, head_dim, n_ctx);
    bmo::RingGeom rg;
    if (registry_geometry(k_cache_dev, &rg)) {
        if (rg.head_dim != head_dim || rg.n_ctx != n_ctx || rg.n_sessions != 1 ||
            rg.n_kv_heads != n_heads || layer >= rg.n_layers)
            return reject("arguments do not match the ring's geometry");
    }
    p.base = static_cast<uint8_t *>(k_cache_dev);
    p.layer = layer;
    p.n_batch = 1;
    p.n_heads = n_heads;
    p.n_kv = n_kv_heads;
    p.pos = pos_dev;
    p.pos_scalar = n_past;
    p.q = q_dev;
    p.k_new = k_dev;
    p.v_new = v_dev;
    p.out = out_dev;
    p.qscale = (1.0f / std::sqrt((float) head_dim)) * kLog2e;
    bmo::launch_decode(p, true, (hipStream_t) stream);
}

}  // extern "C"
