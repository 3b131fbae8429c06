// session.cpp -- the per-session handle of include/bmo_attn.h: the attention
// part of the reference's bmo_handle (src/bmo_api.cpp:164-172).  A handle
// owns one session of a ring, a non-blocking HIP stream, a device-resident
// position that every launch reads (the reference's pos_dev), and a mutex
// that serializes its calls (src/bmo_api.cpp:28, :415).
//
// Two granularities.  A whole token step (forward) runs the fused append +
// attention of every layer at one position and then advances the position
// (h->pos = pos + 1, src/bmo_api.cpp:501).  A model's layer loop
// (src/bmo_compute.cpp:2188-2641) instead interleaves each layer's attention
// with its own work on the handle's stream -- the QKV projection before it,
// the output projection and FFN after it -- so the handle also takes one
// layer at a time (begin_step, layer, end_step), asynchronously.  Either can
// be captured into a HIP graph and replayed per token: capture_begin /
// capture_end bracket whatever the caller enqueues on the handle's stream,
// and the graph reads the position from device memory, so replays keep
// attending (and rotating, with RoPE) at the current position.  A capture
// may start with an asynchronous reset (the depformer's per-frame reset,
// src/bmo_api.cpp:682) and hold several steps (its 8 codebook steps).  This
// is what bmo_capture_graphs / bmo_has_cuda_graphs stand for
// (src/bmo_api.cpp:334-359), whose static capture froze RoPE at the capture
// position and was disabled; the reference keeps per-step depth graphs
// (src/bmo_api.cpp:59-61,535-558).
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
    // what a replay of the graph does to the position: resets it to 0 first
    // (graph_resets) and then advances it graph_adv times
    bool graph_resets = false;
    int graph_adv = 0;
    // an open capture_begin: the position effects recorded so far, and
    // whether a call inside it failed
    bool capturing = false;
    bool cap_resets = false;
    int cap_adv = 0;
    bool cap_failed = false;
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

// The message of the ring call that just failed on this thread (the ring's
// own message could already be another thread's, for a handle on another
// session of the same ring).
std::string ring_message(const char *what) {
    const char *m = bmo::ring_thread_last_error();
    return std::string(what) + ": " + (m && *m ? m : "ring call failed");
}

void drop_graph(bmo_attn_session_t *s) {
    if (s->exec) (void) hipGraphExecDestroy(s->exec);
    if (s->graph) (void) hipGraphDestroy(s->graph);
    s->exec = nullptr;
    s->graph = nullptr;
}

// Queues one layer's fused append + attention at the device position.
// Allocates nothing and synchronizes nothing, so it can be captured.
int enqueue_layer(bmo_attn_session_t *s, int l, const float *q, const float *k, const float *v,
                  float *out, const char *fn) {
    const int rc = s->rope_theta > 0.0f
                       ? bmo_kv_ring_append_decode_rope(s->ring, l, 1, s->dev + 1, s->dev, s->n_heads, q, k,
                                                        v, out, s->scale, s->rope_theta, s->stream)
                       : bmo_kv_ring_append_decode(s->ring, l, 1, s->dev + 1, s->dev, s->n_heads, q, k, v,
                                                   out, s->scale, s->stream);
    if (rc != BMO_ATTN_OK) return fail(s, rc, ring_message(fn));
    return BMO_ATTN_OK;
}

// Queues the position advance that ends a step.
int enqueue_advance(bmo_attn_session_t *s, const char *fn) {
    bmo::launch_advance(s->dev, 1, 1, s->stream);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
    return BMO_ATTN_OK;
}

// Queues one token step on the handle's stream: every layer's fused append +
// attention at the device position, then the position advances by one.
int enqueue_step(bmo_attn_session_t *s, const float *q, const float *k, const float *v, float *out) {
    const int64_t qs = (int64_t) s->n_heads * s->head_dim;
    const int64_t ks = (int64_t) s->n_kv * s->head_dim;
    for (int l = 0; l < s->n_layers; ++l)
        if (int rc = enqueue_layer(s, l, q + l * qs, k + l * ks, v + l * ks, out + l * qs, "token step"))
            return rc;
    return enqueue_advance(s, "token step");
}

// Rejects a call that synchronizes or sets the position from the host while
// a capture is open.
int check_not_capturing(bmo_attn_session_t *s, const char *fn) {
    if (s->capturing)
        return fail(s, BMO_ATTN_ERR_ARG,
                    std::string(fn) + ": not allowed between bmo_attn_session_capture_begin and _end");
    return BMO_ATTN_OK;
}

// Instantiates a finished capture; the previous graph is replaced only when
// this succeeds.
int keep_graph(bmo_attn_session_t *s, hipGraph_t graph, bool resets, int adv, const char *fn) {
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void) hipGraphDestroy(graph);
        return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": instantiate: " + hipGetErrorString(e));
    }
    drop_graph(s);
    s->graph = graph;
    s->exec = exec;
    s->graph_resets = resets;
    s->graph_adv = adv;
    s->last_error.clear();
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

// Waits for the queued work; the position is then next_pos.
int finish(bmo_attn_session_t *s, int64_t next_pos, const char *fn) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
    s->pos = next_pos;
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
        if (s->capturing) {  // an open capture: close it and discard what it recorded
            hipGraph_t graph = nullptr;
            (void) hipStreamEndCapture(s->stream, &graph);
            if (graph) (void) hipGraphDestroy(graph);
            s->capturing = false;
        }
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
    const char *fn = "bmo_attn_session_reset";
    try {
        if (int rc = check_not_capturing(s, fn)) return rc;
        DeviceGuard dg(s->device);
        const int rc = bmo_kv_ring_reset(s->ring, s->session, s->stream);
        if (rc != BMO_ATTN_OK) return fail(s, rc, ring_message(fn));
        bmo::launch_set_pos(s->dev, 0, s->stream);
        return finish(s, 0, fn);
    } catch (...) {
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
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
        if (int rc = check_not_capturing(s, fn)) return rc;
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
        return finish(s, (int64_t) pos + 1, fn);
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
        if (int rc = check_not_capturing(s, fn)) return rc;
        if (!q || !k || !v || !out) return fail(s, BMO_ATTN_ERR_NULL, std::string(fn) + ": null pointer argument");
        DeviceGuard dg(s->device);
        hipError_t e = hipStreamSynchronize(s->stream);
        if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
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
        return keep_graph(s, graph, false, 1, fn);
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
        if (int rc = check_not_capturing(s, fn)) return rc;
        if (!s->exec) return fail(s, BMO_ATTN_ERR_ARG, std::string(fn) + ": no captured step (call bmo_attn_session_capture first)");
        if (int rc = check_pos(s, pos, fn)) return rc;
        if (!s->graph_resets && (int64_t) pos + s->graph_adv > INT_MAX)
            return fail(s, BMO_ATTN_ERR_ARG, std::string(fn) + ": the graph's steps would pass 2^31 - 1");
        DeviceGuard dg(s->device);
        if (!s->graph_resets) seek(s, pos);
        const hipError_t e = hipGraphLaunch(s->exec, s->stream);
        if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
        return finish(s, (s->graph_resets ? 0 : (int64_t) pos) + s->graph_adv, fn);
    } catch (...) {
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

int bmo_attn_session_begin_step(bmo_attn_session_t *s, int pos) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    const char *fn = "bmo_attn_session_begin_step";
    try {
        if (int rc = check_not_capturing(s, fn)) return rc;
        if (int rc = check_pos(s, pos, fn)) return rc;
        DeviceGuard dg(s->device);
        seek(s, pos);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
        s->pos = pos;
        s->last_error.clear();
        return BMO_ATTN_OK;
    } catch (...) {
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

int bmo_attn_session_layer(bmo_attn_session_t *s, int layer, const float *q, const float *k,
                           const float *v, float *out) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    const char *fn = "bmo_attn_session_layer";
    try {
        int rc = BMO_ATTN_OK;
        if (!q || !k || !v || !out)
            rc = fail(s, BMO_ATTN_ERR_NULL, std::string(fn) + ": null pointer argument");
        else if (layer < 0 || layer >= s->n_layers)
            rc = fail(s, BMO_ATTN_ERR_ARG, std::string(fn) + ": layer out of range");
        else {
            DeviceGuard dg(s->device);
            rc = enqueue_layer(s, layer, q, k, v, out, fn);
        }
        if (rc != BMO_ATTN_OK) {
            s->cap_failed = s->capturing;
            return rc;
        }
        s->last_error.clear();
        return BMO_ATTN_OK;
    } catch (...) {
        s->cap_failed = s->capturing;
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

int bmo_attn_session_end_step(bmo_attn_session_t *s) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    const char *fn = "bmo_attn_session_end_step";
    try {
        const int64_t next = (s->capturing ? (s->cap_resets ? 0 : s->pos) + s->cap_adv : s->pos) + 1;
        if (next > INT_MAX) {
            s->cap_failed = s->capturing;
            return fail(s, BMO_ATTN_ERR_ARG, std::string(fn) + ": the position would pass 2^31 - 1");
        }
        DeviceGuard dg(s->device);
        if (int rc = enqueue_advance(s, fn)) {
            s->cap_failed = s->capturing;
            return rc;
        }
        if (s->capturing)
            ++s->cap_adv;
        else
            s->pos = next;
        s->last_error.clear();
        return BMO_ATTN_OK;
    } catch (...) {
        s->cap_failed = s->capturing;
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

int bmo_attn_session_reset_async(bmo_attn_session_t *s) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    const char *fn = "bmo_attn_session_reset_async";
    try {
        DeviceGuard dg(s->device);
        const int rc = bmo_kv_ring_reset(s->ring, s->session, s->stream);
        if (rc != BMO_ATTN_OK) {
            s->cap_failed = s->capturing;
            return fail(s, rc, ring_message(fn));
        }
        bmo::launch_set_pos(s->dev, 0, s->stream);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            s->cap_failed = s->capturing;
            return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
        }
        if (s->capturing) {
            s->cap_resets = true;
            s->cap_adv = 0;
        } else {
            s->pos = 0;
        }
        s->last_error.clear();
        return BMO_ATTN_OK;
    } catch (...) {
        s->cap_failed = s->capturing;
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

int bmo_attn_session_sync(bmo_attn_session_t *s) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    const char *fn = "bmo_attn_session_sync";
    try {
        if (int rc = check_not_capturing(s, fn)) return rc;
        DeviceGuard dg(s->device);
        return finish(s, s->pos, fn);
    } catch (...) {
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

int bmo_attn_session_capture_begin(bmo_attn_session_t *s) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    const char *fn = "bmo_attn_session_capture_begin";
    try {
        if (int rc = check_not_capturing(s, fn)) return rc;
        DeviceGuard dg(s->device);
        hipError_t e = hipStreamSynchronize(s->stream);
        if (e == hipSuccess) e = hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": " + hipGetErrorString(e));
        s->capturing = true;
        s->cap_resets = false;
        s->cap_adv = 0;
        s->cap_failed = false;
        s->last_error.clear();
        return BMO_ATTN_OK;
    } catch (...) {
        return fail(s, BMO_ATTN_ERR_INTERNAL, std::string(fn) + ": unknown exception");
    }
}

int bmo_attn_session_capture_end(bmo_attn_session_t *s) {
    if (!s) return BMO_ATTN_ERR_NULL;
    std::lock_guard<std::mutex> lk(s->mu);
    const char *fn = "bmo_attn_session_capture_end";
    try {
        if (!s->capturing) return fail(s, BMO_ATTN_ERR_ARG, std::string(fn) + ": no capture is open");
        DeviceGuard dg(s->device);
        hipGraph_t graph = nullptr;
        const hipError_t e = hipStreamEndCapture(s->stream, &graph);
        s->capturing = false;
        if (s->cap_failed) {
            if (graph) (void) hipGraphDestroy(graph);
            return fail(s, BMO_ATTN_ERR_ARG, std::string(fn) + ": a call inside the capture failed; the "
                                                               "previous graph is kept");
        }
        if (e != hipSuccess || !graph) {
            if (graph) (void) hipGraphDestroy(graph);
            return fail(s, BMO_ATTN_ERR_HIP, std::string(fn) + ": end capture: " + hipGetErrorString(e));
        }
        return keep_graph(s, graph, s->cap_resets, s->cap_adv, fn);
    } catch (...) {
        s->capturing = false;
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
