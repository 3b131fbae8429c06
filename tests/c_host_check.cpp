// c_host_check.cpp -- a C++ host that drives the library through
// include/bmo_attn.h alone (the HIP runtime only for its device buffers), the
// way the reference's C++ engine drives its attention node: a two-layer ring
// with two sessions, a per-session handle on session 1, and token steps at
// consecutive positions that wrap the ring -- eager whole steps
// (bmo_attn_session_forward), replays of a captured step
// (bmo_attn_session_capture / _replay), eager steps one layer at a time
// (bmo_attn_session_begin_step / _layer / _end_step / _sync, the calls a
// model's layer loop makes between its own kernels), and replays of such a
// step captured by bmo_attn_session_capture_begin / _end -- with and without
// RoPE.  After every step each layer's output is checked against the CPU
// oracle (oracle/liboracle.so, test infrastructure) at
// |gpu - ref| <= 2e-3 + 1e-3 |ref|; at the end the ring's blocks of both
// layers are compared with the oracle's bit for bit.  Prints "ok ..." and
// exits 0, or prints the first failure and exits 1.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "bmo_attn.h"
#include "oracle.h"

namespace {

constexpr int kLayers = 2, kSessions = 2, kSession = 1, kHeads = 8, kKv = 4, kD = 128, kCtx = 48;
// steps [0, 25) forward, [25, 45) replays of a captured step, [45, 52)
// layer by layer, [52, 75) replays of a step captured layer by layer
constexpr int kSteps = 75, kEagerSteps = 25, kReplayEnd = 45, kLayerEnd = 52;
constexpr int kBlocks = kD / 32;

bool hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    std::printf("FAIL %s: %s\n", what, hipGetErrorString(e));
    return false;
}

struct Layer {
    std::vector<orc_block_q4_0> kc, vc;  // oracle ring of this layer, [kv][slot][block]
    // the zero state, as the library's: every byte 0 (d = 0)
    Layer() : kc((size_t) kKv * kCtx * kBlocks), vc((size_t) kKv * kCtx * kBlocks) {}
};

int run(float theta) {
    bmo_kv_ring_t *ring = bmo_kv_ring_create(kLayers, kSessions, kKv, kD, kCtx);
    if (!ring) {
        std::printf("FAIL ring create: %s\n", bmo_kv_ring_last_error(nullptr));
        return 1;
    }
    bmo_attn_session_t *s = bmo_attn_session_create(ring, kSession, kHeads, 0.0f, theta);
    if (!s) {
        std::printf("FAIL session create: %s\n", bmo_attn_session_last_error(nullptr));
        bmo_kv_ring_free(ring);
        return 1;
    }
    const size_t qn = (size_t) kLayers * kHeads * kD, kn = (size_t) kLayers * kKv * kD;
    float *q = nullptr, *k = nullptr, *v = nullptr, *out = nullptr;
    if (!hip_ok(hipMalloc(&q, qn * 4), "hipMalloc") || !hip_ok(hipMalloc(&k, kn * 4), "hipMalloc") ||
        !hip_ok(hipMalloc(&v, kn * 4), "hipMalloc") || !hip_ok(hipMalloc(&out, qn * 4), "hipMalloc"))
        return 1;
    std::vector<Layer> ref(kLayers);
    std::vector<float> hq(qn), hk(kn), hv(kn), hout(qn), rq(kHeads * kD), rk(kKv * kD);
    std::vector<double> want(kHeads * kD);
    const double scale = 1.0 / std::sqrt((double) kD);
    long checked = 0;
    int fails = 0;
    for (int p = 0; p < kSteps && !fails; ++p) {
        const uint64_t seed = 0xC0FFEE00u + (uint64_t) p * 7919u + (theta > 0.0f ? 1u : 0u);
        orc_fill_normal(seed, 0, hq.data(), (int64_t) qn);
        orc_fill_normal(seed, qn, hk.data(), (int64_t) kn);
        orc_fill_normal(seed, qn + kn, hv.data(), (int64_t) kn);
        if (!hip_ok(hipMemcpy(q, hq.data(), qn * 4, hipMemcpyHostToDevice), "hipMemcpy") ||
            !hip_ok(hipMemcpy(k, hk.data(), kn * 4, hipMemcpyHostToDevice), "hipMemcpy") ||
            !hip_ok(hipMemcpy(v, hv.data(), kn * 4, hipMemcpyHostToDevice), "hipMemcpy"))
            return 1;
        // one layer's q/k/v/out inside the step's buffers
        auto layer_call = [&](int l) {
            return bmo_attn_session_layer(s, l, q + (size_t) l * kHeads * kD, k + (size_t) l * kKv * kD,
                                          v + (size_t) l * kKv * kD, out + (size_t) l * kHeads * kD);
        };
        int rc = BMO_ATTN_OK;
        if (p < kEagerSteps) {
            rc = bmo_attn_session_forward(s, p, q, k, v, out);
        } else if (p < kReplayEnd) {
            if (p == kEagerSteps && (rc = bmo_attn_session_capture(s, q, k, v, out)) != BMO_ATTN_OK) {
                std::printf("FAIL capture: %s\n", bmo_attn_session_last_error(s));
                return 1;
            }
            rc = bmo_attn_session_replay(s, p);
        } else if (p < kLayerEnd) {
            rc = bmo_attn_session_begin_step(s, p);
            for (int l = kLayers - 1; l >= 0 && rc == BMO_ATTN_OK; --l) rc = layer_call(l);  // any order
            if (rc == BMO_ATTN_OK) rc = bmo_attn_session_end_step(s);
            if (rc == BMO_ATTN_OK) rc = bmo_attn_session_sync(s);
        } else {
            if (p == kLayerEnd) {
                rc = bmo_attn_session_capture_begin(s);
                for (int l = 0; l < kLayers && rc == BMO_ATTN_OK; ++l) rc = layer_call(l);
                if (rc == BMO_ATTN_OK) rc = bmo_attn_session_end_step(s);
                const int rc_end = bmo_attn_session_capture_end(s);
                if (rc != BMO_ATTN_OK || rc_end != BMO_ATTN_OK) {
                    std::printf("FAIL layer capture: %s\n", bmo_attn_session_last_error(s));
                    return 1;
                }
                if (bmo_attn_session_pos(s) != p) {
                    std::printf("FAIL layer capture moved the position to %lld\n",
                                (long long) bmo_attn_session_pos(s));
                    return 1;
                }
            }
            rc = bmo_attn_session_replay(s, p);
        }
        if (rc != BMO_ATTN_OK) {
            std::printf("FAIL step %d: rc %d: %s\n", p, rc, bmo_attn_session_last_error(s));
            return 1;
        }
        if (bmo_attn_session_pos(s) != p + 1) {
            std::printf("FAIL step %d: handle position %lld\n", p, (long long) bmo_attn_session_pos(s));
            return 1;
        }
        if (!hip_ok(hipMemcpy(hout.data(), out, qn * 4, hipMemcpyDeviceToHost), "hipMemcpy")) return 1;
        for (int l = 0; l < kLayers && !fails; ++l) {
            const float *lq = hq.data() + (size_t) l * kHeads * kD;
            const float *lk = hk.data() + (size_t) l * kKv * kD;
            const float *lv = hv.data() + (size_t) l * kKv * kD;
            if (theta > 0.0f) {
                orc_rope_interleaved(lq, rq.data(), kHeads, kD, p, theta);
                orc_rope_interleaved(lk, rk.data(), kKv, kD, p, theta);
                lq = rq.data();
                lk = rk.data();
            }
            orc_ring_append(ref[l].kc.data(), ref[l].vc.data(), kKv, kD, kCtx, p, lk, lv);
            orc_ring_decode_f64(ref[l].kc.data(), ref[l].vc.data(), kHeads, kKv, kD, kCtx, p, lq, scale,
                                want.data());
            for (int i = 0; i < kHeads * kD; ++i) {
                const double got = hout[(size_t) l * kHeads * kD + i];
                ++checked;
                if (!(std::fabs(got - want[i]) <= 2e-3 + 1e-3 * std::fabs(want[i]))) {
                    std::printf("FAIL theta %g step %d layer %d element %d: got %.7g want %.7g\n", theta, p, l,
                                i, got, want[i]);
                    fails = 1;
                    break;
                }
            }
        }
    }
    // the ring's blocks against the oracle's, both layers, K and V
    std::vector<uint8_t> blocks((size_t) kCtx * kKv * kBlocks * sizeof(orc_block_q4_0));
    for (int l = 0; l < kLayers && !fails; ++l)
        for (int which = 0; which < 2 && !fails; ++which) {
            const int64_t n = bmo_kv_ring_export_q4_0(ring, l, kSession, which, 0, kCtx, blocks.data(),
                                                      (int64_t) blocks.size());
            if (n != (int64_t) blocks.size()) {
                std::printf("FAIL export layer %d: %lld\n", l, (long long) n);
                fails = 1;
                break;
            }
            const std::vector<orc_block_q4_0> &c = which ? ref[l].vc : ref[l].kc;
            // export layout [slot][kv][block]; the oracle's is [kv][slot][block]
            for (int slot = 0; slot < kCtx && !fails; ++slot)
                for (int h = 0; h < kKv; ++h) {
                    const void *a = blocks.data() + ((size_t) slot * kKv + h) * kBlocks * sizeof(orc_block_q4_0);
                    const void *b = &c[((size_t) h * kCtx + slot) * kBlocks];
                    if (std::memcmp(a, b, kBlocks * sizeof(orc_block_q4_0)) != 0) {
                        std::printf("FAIL ring layer %d %s slot %d kv head %d differs\n", l, which ? "V" : "K",
                                    slot, h);
                        fails = 1;
                        break;
                    }
                }
        }
    (void) hipFree(q);
    (void) hipFree(k);
    (void) hipFree(v);
    (void) hipFree(out);
    bmo_attn_session_free(s);
    bmo_kv_ring_free(ring);
    if (!fails)
        std::printf("ok theta %g: %d steps (%d eager, %d replays of a captured step, %d layer by layer, %d "
                    "replays of a step captured layer by layer), %ld values checked, ring bit-exact\n",
                    theta, kSteps, kEagerSteps, kReplayEnd - kEagerSteps, kLayerEnd - kReplayEnd,
                    kSteps - kLayerEnd, checked);
    return fails;
}

}  // namespace

int main() {
    int device_count = 0;
    if (hipGetDeviceCount(&device_count) != hipSuccess || device_count < 1) {
        std::printf("FAIL no HIP device\n");
        return 1;
    }
    if (run(0.0f) != 0) return 1;
    if (run(10000.0f) != 0) return 1;
    return 0;
}
