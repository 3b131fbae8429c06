// session.cpp -- the per-session handle of include/bmo_attn.h: the attention
// part of the reference's bmo_handle (src/bmo_api.cpp:164-172).  A handle
// owns one session of a ring, a non-blocking HIP stream, a device-resident
// position that every launch reads (the reference's pos_dev), and a mutex
// that serializes its calls (src/bmo_api.cpp:28, :415).  A token step runs
// the fused append + attention of every layer at one position and then
// advances the position (h->pos = pos + 1, src/bmo_api.cpp:501).  The step
// can be captured once into a HIP graph and replayed per token: the graph
// reads the position from device memory and ends by advancing it, so
// replays keep attending (and rotating, with RoPE) at the current position.
// This is what bmo_capture_graphs / bmo_has_cuda_graphs stand for
// (src/bmo_api.cpp:334-359), whose static capture froze RoPE at the capture
// position and was disabled.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdio>
#include <exception>
#include <mutex>
#include <string>

#include "../../include/bmo_attn.h"
#include "kernels.hpp"

struct bmo_attn_session {
    bmo_kv_ring_t *ring = nullptr;
    int session = 0;
    int n_layers = 0, n_kv = 0, head_dim = 0, n_ctx = 0;
    int n_heads = 0;
    float scale = 0.0f;
    float rope_theta = 0.0f;  // 0: no RoPE
    int device = 0;
    hipStream_t stream = nullptr;
    int *dev = nullptr;   // dev[0]: position read by every launch; dev[1]: the session id
    int64_t pos = 0;      // next position; dev[0] holds it once queued work has run
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::mutex mu;
    std::string last_error;
};

namespace {

thread_local std::string t_session_create_error;

struct DeviceGuard {
    int prev = -1;
    bool switched = false;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) switched = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard() {
        if (switched) (void) hipSetDevice(prev);
    }
};

int fail(bmo_attn_session_t *s, int code, const std::string &msg) {
    s->last_error = msg;
    return code;
}

// The ring call's message, or a generic one.
std::string ring_message(bmo_attn_session_t *s, const char *what) {
    const char *m = bmo_kv_ring_last_error(s->ring);
    return std::string(what) + ": " + (m ? m : "ring call failed");
}

void drop_graph(bmo_attn_session_t *s) {
    if (s->exec) (void) hipGraphExecDestroy(s->exec);
    if (s->graph) (void) hipGraphDestroy(s->graph);
    s->exec = nullptr;
    s->graph = nullptr;
}

// Queues one token step on the handle's stream: every layer's fused append +
// attention at the device position, then the position advances by one.
// Allocates nothing and synchronizes nothing, so it can be captured.
int enqueue_step(bmo_attn_session_t *s, const float *q, const float *k, const float *v, float *out) {
    const int64_t qs = (int64_t) s->n_heads * s->head_dim;
    const int64_t ks = (int64_t) s->n_kv * s->head_dim;
    for (int l = 0; l < s->n_layers; ++l) {
        const int rc = s->rope_theta > 0.0f
                           ? bmo_kv_ring_append_decode_rope(s->ring, l, 1, s->dev + 1, s->dev, s->n_heads,
                                                            q + l * qs, k + l * ks, v + l * ks, out + l * qs,
                                                            s->scale, s->rope_theta, s->stream)
                           : bmo_kv_ring_append_decode(s->ring, l, 1, s->dev + 1, s->dev, s->n_heads,
                                                       q + l * qs, k + l * ks, v + l * ks, out + l * qs,
                                                       s->scale, s->stream);
        if (rc != BMO_ATTN_OK) return fail(s, rc, ring_message(s, "token step"));
    }
    bmo::launch_advance(s->dev, 1, 1, s->stream);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string("token step: ") + hipGetErrorString(e));
    return BMO_ATTN_OK;
}

// Checks a caller position; the position after it must still be an int.
int check_pos(bmo_attn_session_t *s, int pos, const char *fn) {
    if (pos < 0 || pos > INT_MAX - 1)
        return fail(s, BMO_ATTN_ERR_ARG, std::string(fn) + ": pos must be in [0, 2^31 - 2]");
    return BMO_ATTN_OK;
}

// Makes the device position equal pos before the next step (a no-op when the
// previous step already left it there).
void seek(bmo_attn_session_t *s, int pos) {
    if (pos != s->pos) bmo::launch_set_pos(s->dev, pos, s->stream);
}

int finish(bmo_attn_session_t *s, int pos, const char *fn) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
    s->pos = (int64_t) pos + 1;
    s->last_error.clear();
    return BMO_ATTN_OK;
}

}  // namespace

extern "C" {

bmo_attn_session_t *bmo_attn_session_create(bmo_kv_ring_t *ring, int session, int n_heads, float scale,
                                            float rope_theta) {
    t_session_create_error.clear();
    auto reject = [](const std::string &m) -> bmo_attn_session_t * {
        t_session_create_error = "bmo_attn_session_create: " + m;
        std::fprintf(stderr, "[bmo_attn] %s\n", t_session_create_error.c_str());
        return nullptr;
    };
    if (!ring) return reject("ring is NULL");
    bmo_attn_session_t *s = nullptr;
    try {
        s = new bmo_attn_session();
        s->ring = ring;
        int n_sessions = 0;
        (void) bmo_kv_ring_geometry(ring, &s->n_layers, &n_sessions, &s->n_kv, &s->head_dim, &s->n_ctx);
        if (session < 0 || session >= n_sessions) {
            delete s;
            return reject("session out of range");
        }
        if (n_heads <= 0 || n_heads % s->n_kv != 0) {
            delete s;
            return reject("n_heads must be a positive multiple of the ring's n_kv_heads");
        }
        if (!(rope_theta >= 0.0f) || !std::isfinite(rope_theta) || !std::isfinite(scale)) {
            delete s;
            return reject("rope_theta must be >= 0 and finite, scale finite");
        }
        s->session = session;
        s->n_heads = n_heads;
        s->scale = scale;
        s->rope_theta = rope_theta;
        hipPointerAttribute_t attr{};
        if (hipPointerGetAttributes(&attr, bmo_kv_ring_k_base(ring)) != hipSuccess) {
            delete s;
            return reject("cannot find the ring's device");
        }
        s->device = attr.device;
        DeviceGuard dg(s->device);
        hipError_t e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipMalloc(&s->dev, 2 * sizeof(int));
        if (e == hipSuccess) {
            bmo::launch_set_pos(s->dev, 0, s->stream);
            e = hipMemcpyAsync(s->dev + 1, &s->session, sizeof(int), hipMemcpyHostToDevice, s->stream);
        }
        if (e == hipSuccess) e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
        if (e != hipSuccess) {
            const std::string m = std::string("HIP setup failed: ") + hipGetErrorString(e);
            if (s->dev) (void) hipFree(s->dev);
            if (s->stream) (void) hipStreamDestroy(s->stream);
            delete s;
            return reject(m);
        }
        return s;
    } catch (const std::exception &ex) {
        delete s;
        return reject(ex.what());
    } catch (...) {
        delete s;
        return reject("unknown exception");
    }
}

void bmo_attn_session_free(bmo_attn_session_t *s) {
    if (!s) return;
    try {
        std::lock_guard<std::mutex> lk(s->mu);
        DeviceGuard dg(s->device);
        if (s->stream) (void) hipStreamSynchronize(s->stream);
        drop_graph(s);
        if (s->dev) (void) hipFree(s->dev);
        if (s->stream) (void) hipStreamDestroy(s->stream);
    } catch (...) {
    }
    delete s;
}

int bmo_attn_session_reset(bmo_attn_session_t *s) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    try {
        DeviceGuard dg(s->device);
        const int rc = bmo_kv_ring_reset(s->ring, s->session, s->stream);
        if (rc != BMO_ATTN_OK) return fail(s, rc, ring_message(s, "bmo_attn_session_reset"));
        bmo::launch_set_pos(s->dev, 0, s->stream);
        const int r = finish(s, -1, "bmo_attn_session_reset");  // next position 0
        return r;
    } catch (...) {
        return fail(s, BMO_ATTN_ERR_INTERNAL, "bmo_attn_session_reset: unknown exception");
    }
}

int64_t bmo_attn_session_pos(bmo_attn_session_t *s) {
    if (!s) return -1;
    std::lock_guard<std::mutex> lk(s->mu);
    return s->pos;
}

void *bmo_attn_session_stream(bmo_attn_session_t *s) { return s ? (void *) s->stream : nullptr; }

int bmo_attn_session_forward(bmo_attn_session_t *s, int pos, const float *q, const float *k,
                             const float *v, float *out) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    const char *fn = "bmo_attn_session_forward";
    try {
        if (!q || !k || !v || !out) return fail(s, BMO_ATTN_ERR_NULL, std::string(fn) + ": null pointer argument");
        if (int rc = check_pos(s, pos, fn)) return rc;
        DeviceGuard dg(s->device);
        seek(s, pos);
        if (int rc = enqueue_step(s, q, k, v, out)) {
            (void) hipStreamSynchronize(s->stream);
            // the device position is unknown after a partial step: set it again
            bmo::launch_set_pos(s->dev, (int) s->pos, s->stream);
            (void) hipStreamSynchronize(s->stream);
            return rc;
        }
        return finish(s, pos, fn);
    } catch (...) {
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

int bmo_attn_session_capture(bmo_attn_session_t *s, const float *q, const float *k, const float *v,
                             float *out) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    const char *fn = "bmo_attn_session_capture";
    try {
        if (!q || !k || !v || !out) return fail(s, BMO_ATTN_ERR_NULL, std::string(fn) + ": null pointer argument");
        DeviceGuard dg(s->device);
        hipError_t e = hipStreamSynchronize(s->stream);
        if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
        drop_graph(s);
        e = hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": begin capture: " + hipGetErrorString(e));
        const int rc = enqueue_step(s, q, k, v, out);
        hipGraph_t graph = nullptr;
        e = hipStreamEndCapture(s->stream, &graph);
        if (rc != BMO_ATTN_OK) {
            if (graph) (void) hipGraphDestroy(graph);
            return rc;
        }
        if (e != hipSuccess || !graph)
            return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": end capture: " + hipGetErrorString(e));
        hipGraphExec_t exec = nullptr;
        e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void) hipGraphDestroy(graph);
            return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": instantiate: " + hipGetErrorString(e));
        }
        s->graph = graph;
        s->exec = exec;
        s->last_error.clear();
        return BMO_ATTN_OK;
    } catch (...) {
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

int bmo_attn_session_has_graph(bmo_attn_session_t *s) {
    if (!s) return 0;
    std::lock_guard<std::mutex> lk(s->mu);
    return s->exec ? 1 : 0;
}

int bmo_attn_session_replay(bmo_attn_session_t *s, int pos) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    const char *fn = "bmo_attn_session_replay";
    try {
        if (!s->exec) return fail(s, BMO_ATTN_ERR_ARG, std::string(fn) + ": no captured step (call bmo_attn_session_capture first)");
        if (int rc = check_pos(s, pos, fn)) return rc;
        DeviceGuard dg(s->device);
        seek(s, pos);
        const hipError_t e = hipGraphLaunch(s->exec, s->stream);
        if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
        return finish(s, pos, fn);
    } catch (...) {
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

const char *bmo_attn_session_last_error(bmo_attn_session_t *s) {
    if (!s) return t_session_create_error.empty() ? nullptr : t_session_create_error.c_str();
    // a copy per thread (see bmo_kv_ring_last_error)
    thread_local std::string t_copy;
    {
        std::lock_guard<std::mutex> lk(s->mu);
        t_copy = s->last_error;
    }
    return t_copy.empty() ? nullptr : t_copy.c_str();
}

}  // extern "C"
