// c_host_kernels.cpp -- a C++ host that calls the library's node-level
// entry points through include/bmo_attn.h alone (the HIP runtime only for
// device buffers), the way the reference's C++ engine calls its kernels:
//   - bmo_launch_decode_attention, the signature of the reference's
//     launch_decode_attention (src/bmo.h:412-426), over a ring allocated as
//     the reference allocates its cache (one session, n_heads head slots):
//     40 token steps at layer 1 of a two-layer, 32-slot ring, the position
//     given as n_past on even steps and through pos_dev on odd ones;
//   - bmo_kv_ring_prefill on two sessions at once, three chunks each (the
//     second wraps the ring), on a ring with one query head per kv head (the
//     one-kernel path) and on one with four query heads per kv head (the
//     staged path);
//   - bmo_launch_gemv_q4_0_q8_1, the arguments of the reference's
//     launch_gemv_q4_0_q8_1 (src/bmo_cuda_kernels.cu:685-711), at a shape
//     each of its two kernels serves, with the Q8_1 scratch requested.
// Attention outputs are checked against the CPU oracle (oracle/liboracle.so,
// test infrastructure) at |gpu - ref| <= 2e-3 + 1e-3 |ref| and the rings'
// blocks bit for bit; GEMV outputs within 1e-5 of the oracle's rounding-error
// scale (plus 1e-6) and the Q8_1 scratch bit for bit.  Prints one "ok ..."
// line per part and exits 0, or prints the first failure and exits 1.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "bmo_attn.h"
#include "oracle.h"

namespace {

bool hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    std::printf("FAIL %s: %s\n", what, hipGetErrorString(e));
    return false;
}

// A device copy of a host vector (freed by the caller).
template <typename T>
T *to_dev(const std::vector<T> &h) {
    void *d = nullptr;
    if (!hip_ok(hipMalloc(&d, h.size() * sizeof(T)), "hipMalloc")) return nullptr;
    if (!hip_ok(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy")) return nullptr;
    return static_cast<T *>(d);
}

bool close_to(double got, double want) { return std::fabs(got - want) <= 2e-3 + 1e-3 * std::fabs(want); }

// The ring's blocks of (layer, session) against an oracle stripe
// ([kv][slot][block]); the export layout is [slot][kv][block].
bool ring_matches(bmo_kv_ring_t *ring, int layer, int session, int n_kv, int head_dim, int n_ctx,
                  const std::vector<orc_block_q4_0> &kc, const std::vector<orc_block_q4_0> &vc, const char *what) {
    const int nb = head_dim / 32;
    std::vector<uint8_t> blocks((size_t) n_ctx * n_kv * nb * sizeof(orc_block_q4_0));
    for (int which = 0; which < 2; ++which) {
        const int64_t n = bmo_kv_ring_export_q4_0(ring, layer, session, which, 0, n_ctx, blocks.data(),
                                                  (int64_t) blocks.size());
        if (n != (int64_t) blocks.size()) {
            std::printf("FAIL %s: export returned %lld\n", what, (long long) n);
            return false;
        }
        const std::vector<orc_block_q4_0> &c = which ? vc : kc;
        for (int slot = 0; slot < n_ctx; ++slot)
            for (int h = 0; h < n_kv; ++h) {
                const void *a = blocks.data() + ((size_t) slot * n_kv + h) * nb * sizeof(orc_block_q4_0);
                if (std::memcmp(a, &c[((size_t) h * n_ctx + slot) * nb], nb * sizeof(orc_block_q4_0)) != 0) {
                    std::printf("FAIL %s: ring session %d %s slot %d kv head %d differs\n", what, session,
                                which ? "V" : "K", slot, h);
                    return false;
                }
            }
    }
    return true;
}

int run_node_launcher() {
    constexpr int kLayers = 2, kLayer = 1, kHeads = 4, kD = 128, kCtx = 32, kSteps = 40, kNb = kD / 32;
    bmo_kv_ring_t *ring = bmo_kv_ring_create(kLayers, 1, kHeads, kD, kCtx);
    if (!ring) {
        std::printf("FAIL node ring create: %s\n", bmo_kv_ring_last_error(nullptr));
        return 1;
    }
    const size_t n = (size_t) kHeads * kD;
    float *q = nullptr, *k = nullptr, *v = nullptr, *out = nullptr;
    int *pos_dev = nullptr;
    if (!hip_ok(hipMalloc(&q, n * 4), "hipMalloc") || !hip_ok(hipMalloc(&k, n * 4), "hipMalloc") ||
        !hip_ok(hipMalloc(&v, n * 4), "hipMalloc") || !hip_ok(hipMalloc(&out, n * 4), "hipMalloc") ||
        !hip_ok(hipMalloc(&pos_dev, 4), "hipMalloc"))
        return 1;
    std::vector<orc_block_q4_0> kc((size_t) kHeads * kCtx * kNb), vc(kc.size());
    std::vector<float> hq(n), hk(n), hv(n), hout(n);
    std::vector<double> want(n);
    int fails = 0;
    for (int p = 0; p < kSteps && !fails; ++p) {
        const uint64_t seed = 0x0DE00000u + (uint64_t) p;
        orc_fill_normal(seed, 0, hq.data(), (int64_t) n);
        orc_fill_normal(seed, n, hk.data(), (int64_t) n);
        orc_fill_normal(seed, 2 * n, hv.data(), (int64_t) n);
        if (!hip_ok(hipMemcpy(q, hq.data(), n * 4, hipMemcpyHostToDevice), "hipMemcpy") ||
            !hip_ok(hipMemcpy(k, hk.data(), n * 4, hipMemcpyHostToDevice), "hipMemcpy") ||
            !hip_ok(hipMemcpy(v, hv.data(), n * 4, hipMemcpyHostToDevice), "hipMemcpy") ||
            !hip_ok(hipMemcpy(pos_dev, &p, 4, hipMemcpyHostToDevice), "hipMemcpy"))
            return 1;
        const bool via_dev = p % 2 == 1;
        bmo_launch_decode_attention(q, k, v, bmo_kv_ring_k_base(ring), bmo_kv_ring_v_base(ring), out, kD, kHeads,
                                    kHeads, kCtx, via_dev ? 0 : p, kLayer, nullptr, via_dev ? pos_dev : nullptr);
        if (!hip_ok(hipGetLastError(), "launch") || !hip_ok(hipDeviceSynchronize(), "sync") ||
            !hip_ok(hipMemcpy(hout.data(), out, n * 4, hipMemcpyDeviceToHost), "hipMemcpy"))
            return 1;
        orc_ring_append(kc.data(), vc.data(), kHeads, kD, kCtx, p, hk.data(), hv.data());
        orc_ring_decode_f64(kc.data(), vc.data(), kHeads, kHeads, kD, kCtx, p, hq.data(), 1.0 / std::sqrt((double) kD),
                            want.data());
        for (size_t i = 0; i < n; ++i)
            if (!close_to(hout[i], want[i])) {
                std::printf("FAIL node step %d element %zu: got %.7g want %.7g\n", p, i, (double) hout[i], want[i]);
                fails = 1;
                break;
            }
    }
    if (!fails && !ring_matches(ring, kLayer, 0, kHeads, kD, kCtx, kc, vc, "node")) fails = 1;
    (void) hipFree(q);
    (void) hipFree(k);
    (void) hipFree(v);
    (void) hipFree(out);
    (void) hipFree(pos_dev);
    bmo_kv_ring_free(ring);
    if (!fails)
        std::printf("ok node launcher: %d steps (pos as n_past and through pos_dev), ring bit-exact\n", kSteps);
    return fails;
}

int run_prefill(int n_kv, int n_heads) {
    constexpr int kSessions = 2, kD = 128, kCtx = 64, kNb = kD / 32;
    struct Call {
        int sids[2], pos0[2], n_tok;
    };
    // the second call of each session wraps the ring; the third starts past it
    const Call calls[] = {{{0, 1}, {0, 0}, 40}, {{1, 0}, {40, 40}, 50}, {{0, 1}, {90, 90}, 64}};
    bmo_kv_ring_t *ring = bmo_kv_ring_create(1, kSessions, n_kv, kD, kCtx);
    if (!ring) {
        std::printf("FAIL prefill ring create: %s\n", bmo_kv_ring_last_error(nullptr));
        return 1;
    }
    std::vector<std::vector<orc_block_q4_0>> kc(kSessions, std::vector<orc_block_q4_0>((size_t) n_kv * kCtx * kNb));
    std::vector<std::vector<orc_block_q4_0>> vc = kc;
    const double scale = 1.0 / std::sqrt((double) kD);
    int fails = 0, ci = 0;
    long checked = 0;
    for (const Call &c : calls) {
        const int nt = c.n_tok;
        const size_t qn = (size_t) nt * n_heads * kD, kn = (size_t) nt * n_kv * kD;
        // bf16 inputs: the oracle takes their fp32 values, the library their bits
        std::vector<float> fq(2 * qn), fk(2 * kn), fv(2 * kn);
        const uint64_t seed = 0x9F000000u + 17u * (uint64_t) ci + (uint64_t) n_heads;
        orc_fill_normal(seed, 0, fq.data(), (int64_t) fq.size());
        orc_fill_normal(seed, fq.size(), fk.data(), (int64_t) fk.size());
        orc_fill_normal(seed, fq.size() + fk.size(), fv.data(), (int64_t) fv.size());
        std::vector<uint16_t> bq(fq.size()), bk(fk.size()), bv(fv.size());
        auto to_bf16 = [](std::vector<float> &f, std::vector<uint16_t> &b) {
            for (size_t i = 0; i < f.size(); ++i) {
                f[i] = orc_round_bf16(f[i]);
                uint32_t u;
                std::memcpy(&u, &f[i], 4);
                b[i] = (uint16_t) (u >> 16);
            }
        };
        to_bf16(fq, bq);
        to_bf16(fk, bk);
        to_bf16(fv, bv);
        std::vector<int> sids(c.sids, c.sids + 2), pos0(c.pos0, c.pos0 + 2);
        uint16_t *dq = to_dev(bq), *dk = to_dev(bk), *dv = to_dev(bv);
        int *dsid = to_dev(sids), *dpos = to_dev(pos0);
        float *dout = nullptr;
        if (!dq || !dk || !dv || !dsid || !dpos || !hip_ok(hipMalloc(&dout, 2 * qn * 4), "hipMalloc")) return 1;
        const int rc = bmo_kv_ring_prefill(ring, 0, 2, dsid, dpos, nt, n_heads, dq, dk, dv, dout, 0.0f, nullptr);
        std::vector<float> hout(2 * qn);
        if (rc != BMO_ATTN_OK) {
            std::printf("FAIL prefill call %d: rc %d: %s\n", ci, rc, bmo_kv_ring_last_error(ring));
            return 1;
        }
        if (!hip_ok(hipDeviceSynchronize(), "sync") ||
            !hip_ok(hipMemcpy(hout.data(), dout, hout.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy"))
            return 1;
        std::vector<double> want(qn);
        for (int b = 0; b < 2 && !fails; ++b) {
            const int s = c.sids[b];
            orc_ring_prefill_f64(kc[s].data(), vc[s].data(), n_heads, n_kv, kD, kCtx, c.pos0[b], nt,
                                 fq.data() + b * qn, fk.data() + b * kn, fv.data() + b * kn, scale, want.data());
            for (size_t i = 0; i < qn; ++i, ++checked)
                if (!close_to(hout[b * qn + i], want[i])) {
                    std::printf("FAIL prefill heads %d/%d call %d entry %d element %zu: got %.7g want %.7g\n", n_heads,
                                n_kv, ci, b, i, (double) hout[b * qn + i], want[i]);
                    fails = 1;
                    break;
                }
        }
        (void) hipFree(dq);
        (void) hipFree(dk);
        (void) hipFree(dv);
        (void) hipFree(dsid);
        (void) hipFree(dpos);
        (void) hipFree(dout);
        if (fails) break;
        ++ci;
    }
    for (int s = 0; s < kSessions && !fails; ++s)
        if (!ring_matches(ring, 0, s, n_kv, kD, kCtx, kc[s], vc[s], "prefill")) fails = 1;
    bmo_kv_ring_free(ring);
    if (!fails)
        std::printf("ok prefill %d query heads on %d kv heads: 3 chunks x 2 sessions, %ld values checked, ring "
                    "bit-exact\n",
                    n_heads, n_kv, checked);
    return fails;
}

int run_gemv(int rows, int cols) {
    const int nb = cols / 32;
    std::vector<float> w((size_t) rows * cols), x(cols);
    orc_fill_normal(0x6E000000u + (uint64_t) cols, 0, w.data(), (int64_t) w.size());
    orc_fill_normal(0x6E100000u + (uint64_t) cols, 0, x.data(), (int64_t) x.size());
    std::vector<orc_block_q4_0> wq((size_t) rows * nb);
    for (int r = 0; r < rows; ++r) orc_quantize_row_q4_0(w.data() + (size_t) r * cols, wq.data() + (size_t) r * nb, cols);
    std::vector<orc_block_q8_1> xq(nb);
    orc_quantize_row_q8_1_bmo(x.data(), xq.data(), cols);
    std::vector<double> want(rows), tabs(rows);
    orc_gemv_q4_0_q8_1_f64(wq.data(), xq.data(), rows, cols, want.data());
    orc_gemv_term_abs_f64(wq.data(), xq.data(), rows, cols, tabs.data());
    orc_block_q4_0 *dw = to_dev(wq);
    float *dx = to_dev(x), *dy = nullptr;
    void *scratch = nullptr;
    if (!dw || !dx || !hip_ok(hipMalloc(&dy, (size_t) rows * 4), "hipMalloc") ||
        !hip_ok(hipMalloc(&scratch, (size_t) nb * sizeof(orc_block_q8_1)), "hipMalloc"))
        return 1;
    const int rc = bmo_launch_gemv_q4_0_q8_1(dw, dx, dy, rows, cols, scratch, nullptr);
    std::vector<float> y(rows);
    std::vector<orc_block_q8_1> got_q(nb);
    int fails = 0;
    if (rc != BMO_ATTN_OK) {
        std::printf("FAIL gemv %dx%d: rc %d\n", rows, cols, rc);
        fails = 1;
    } else if (!hip_ok(hipDeviceSynchronize(), "sync") ||
               !hip_ok(hipMemcpy(y.data(), dy, y.size() * 4, hipMemcpyDeviceToHost), "hipMemcpy") ||
               !hip_ok(hipMemcpy(got_q.data(), scratch, got_q.size() * sizeof(orc_block_q8_1), hipMemcpyDeviceToHost),
                       "hipMemcpy")) {
        return 1;
    } else {
        if (std::memcmp(got_q.data(), xq.data(), got_q.size() * sizeof(orc_block_q8_1)) != 0) {
            std::printf("FAIL gemv %dx%d: Q8_1 scratch differs from the oracle's blocks\n", rows, cols);
            fails = 1;
        }
        for (int r = 0; r < rows && !fails; ++r)
            if (!(std::fabs(y[r] - want[r]) <= 1e-5 * tabs[r] + 1e-6)) {
                std::printf("FAIL gemv %dx%d row %d: got %.9g want %.9g\n", rows, cols, r, (double) y[r], want[r]);
                fails = 1;
            }
    }
    (void) hipFree(dw);
    (void) hipFree(dx);
    (void) hipFree(dy);
    (void) hipFree(scratch);
    if (!fails) std::printf("ok gemv %dx%d: rows within tolerance, Q8_1 scratch bit-exact\n", rows, cols);
    return fails;
}

}  // namespace

int main() {
    int device_count = 0;
    if (hipGetDeviceCount(&device_count) != hipSuccess || device_count < 1) {
        std::printf("FAIL no HIP device\n");
        return 1;
    }
    if (run_node_launcher() != 0) return 1;
    if (run_prefill(4, 4) != 0) return 1;   // one query head per kv head: one kernel
    if (run_prefill(2, 8) != 0) return 1;   // four per kv head: stage, attention, commit
    if (run_gemv(1000, 4096) != 0) return 1;  // the streaming kernel
    if (run_gemv(77, 192) != 0) return 1;     // the pair-walking kernel (cols not a multiple of 256)
    return 0;
}
