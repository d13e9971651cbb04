// A caller of libdashmi that binds nothing but include/dashmi.h: device buffers, copies and the
// operations go through the C ABI alone, as a Rust -sys crate (or any FFI) would drive it. Each
// check runs a small call whose result has a closed form and compares it in double precision:
//   attention with q = 0: every visible key scores the same, so o[i] is the mean of the visible
//     values, lse[i] = ln(visible count), and (backward) dk = 0, dv[j] = sum over the rows i that
//     see j of dO[i] / count(i), dq[i] = scale / count(i) sum_j (dO[i] . (v[j] - o[i])) k[j];
//   decode with q = 0: the mean of each sequence's cached values;
//   the recurrent step from a zero state: S = beta k v^T, out = beta scale (k . q) v.
// Exit status 0 when every check passes. Run by tests/test_gpu_host_check.py.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "dashmi.h"

namespace {

uint16_t to_bf16(float x) {  // round to nearest even (the values used here are exact)
    uint32_t u;
    std::memcpy(&u, &x, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float from_bf16(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float x;
    std::memcpy(&x, &u, 4);
    return x;
}

int failures = 0;

void check(const char *what, double err, double tol) {
    const bool ok = err <= tol;
    std::printf("%-44s max error %.3e (bound %.1e) %s\n", what, err, tol, ok ? "ok" : "FAIL");
    if (!ok) failures++;
}

#define CALL(x)                                                                         \
    do {                                                                                \
        const int rc_ = (x);                                                            \
        if (rc_ != DM_OK) {                                                             \
            std::printf("%s failed (%d): %s\n", #x, rc_, dm_last_error());              \
            return 1;                                                                   \
        }                                                                               \
    } while (0)

// a device copy of a host vector
template <typename T>
void *upload(const std::vector<T> &h) {
    void *p = nullptr;
    if (dm_device_alloc(h.size() * sizeof(T), &p) != DM_OK) return nullptr;
    if (dm_copy_to_device(p, h.data(), h.size() * sizeof(T), nullptr) != DM_OK) return nullptr;
    return p;
}

template <typename T>
std::vector<T> download(const void *p, size_t n) {
    std::vector<T> h(n);
    dm_copy_to_host(h.data(), p, n * sizeof(T), nullptr);
    return h;
}

int attention_check() {
    const int64_t T = 300, Hq = 4, Hkv = 2, D = 128, G = Hq / Hkv;
    std::vector<uint16_t> q(T * Hq * D, to_bf16(0.f)), k(T * Hkv * D), v(T * Hkv * D),
        dO(T * Hq * D);
    for (int64_t j = 0; j < T; j++)
        for (int64_t h = 0; h < Hkv; h++)
            for (int64_t d = 0; d < D; d++) {
                k[(j * Hkv + h) * D + d] = to_bf16((float)((j * 5 + d * 11 + h) % 9) - 4.f);
                v[(j * Hkv + h) * D + d] = to_bf16((float)((j * 7 + d * 3 + h) % 17) - 8.f);
            }
    for (int64_t i = 0; i < T; i++)
        for (int64_t h = 0; h < Hq; h++)
            for (int64_t d = 0; d < D; d++)
                dO[(i * Hq + h) * D + d] = to_bf16(0.25f * (float)((i * 3 + d + 2 * h) % 7 - 3));
    dm_attention_desc desc;
    std::memset(&desc, 0, sizeof(desc));
    desc.b = 1, desc.tq = T, desc.tk = T, desc.hq = Hq, desc.hkv = Hkv, desc.d = D;
    desc.dtype = DM_BF16, desc.mask_kind = DM_MASK_NONE;
    desc.options.causal = 1, desc.options.deterministic = 1;
    desc.options.window_left = desc.options.window_right = DM_UNBOUNDED;
    const double scale = 1.0 / std::sqrt((double)D);

    void *dq_ = upload(q), *dk_ = upload(k), *dv_ = upload(v), *ddo = upload(dO);
    void *o = nullptr, *lse = nullptr, *gq = nullptr, *gk = nullptr, *gv = nullptr, *ws = nullptr;
    CALL(dm_device_alloc(q.size() * 2, &o));
    CALL(dm_device_alloc(T * Hq * 4, &lse));
    CALL(dm_device_alloc(q.size() * 2, &gq));
    CALL(dm_device_alloc(k.size() * 2, &gk));
    CALL(dm_device_alloc(v.size() * 2, &gv));
    const size_t wsb = std::max(dm_attention_fwd_workspace(&desc), dm_attention_bwd_workspace(&desc));
    CALL(dm_device_alloc(wsb, &ws));
    dm_probe_reset();
    CALL(dm_attention_fwd(&desc, dq_, dk_, dv_, o, (float *)lse, ws, wsb, nullptr));
    CALL(dm_attention_bwd(&desc, dq_, dk_, dv_, o, (const float *)lse, ddo, gq, gk, gv, ws, wsb,
                          nullptr));
    CALL(dm_stream_synchronize(nullptr));
    const bool mfma = dm_probe_count(DM_PROBE_ATTN_FWD_MFMA) > 0 && dm_probe_count(DM_PROBE_ATTN_BWD_MFMA) > 0;
    std::printf("attention ran on the MFMA kernels: %s\n", mfma ? "yes" : "NO");
    if (!mfma) failures++;
    const auto ho = download<uint16_t>(o, q.size());
    const auto hl = download<float>(lse, T * Hq);
    const auto hgq = download<uint16_t>(gq, q.size());
    const auto hgk = download<uint16_t>(gk, k.size());
    const auto hgv = download<uint16_t>(gv, v.size());

    auto V = [&](int64_t j, int64_t kh, int64_t d) { return (double)from_bf16(v[(j * Hkv + kh) * D + d]); };
    auto K = [&](int64_t j, int64_t kh, int64_t d) { return (double)from_bf16(k[(j * Hkv + kh) * D + d]); };
    auto DO = [&](int64_t i, int64_t h, int64_t d) { return (double)from_bf16(dO[(i * Hq + h) * D + d]); };
    double eo = 0, el = 0, eq = 0, ek = 0, ev = 0, mo = 0, mq = 0, mv = 0;
    std::vector<double> ob(D), gvd(T * Hkv * D, 0.0);
    for (int64_t i = 0; i < T; i++)
        for (int64_t h = 0; h < Hq; h++) {
            const int64_t kh = h / G, n = i + 1;
            for (int64_t d = 0; d < D; d++) {
                double s = 0;
                for (int64_t j = 0; j <= i; j++) s += V(j, kh, d);
                ob[d] = s / n;
                eo = std::max(eo, std::fabs(ob[d] - from_bf16(ho[(i * Hq + h) * D + d])));
                mo = std::max(mo, std::fabs(ob[d]));
            }
            el = std::max(el, std::fabs(std::log((double)n) - hl[i * Hq + h]));
            // dq[i] = scale / n sum_j (dO[i] . (v[j] - o[i])) k[j]; dv[j] += dO[i] / n
            double doo = 0;
            for (int64_t d = 0; d < D; d++) doo += DO(i, h, d) * ob[d];
            std::vector<double> g(D, 0.0);
            for (int64_t j = 0; j <= i; j++) {
                double dv_ = 0;
                for (int64_t d = 0; d < D; d++) dv_ += DO(i, h, d) * V(j, kh, d);
                const double w = scale * (dv_ - doo) / n;
                for (int64_t d = 0; d < D; d++) {
                    g[d] += w * K(j, kh, d);
                    gvd[(j * Hkv + kh) * D + d] += DO(i, h, d) / n;
                }
            }
            for (int64_t d = 0; d < D; d++) {
                eq = std::max(eq, std::fabs(g[d] - from_bf16(hgq[(i * Hq + h) * D + d])));
                mq = std::max(mq, std::fabs(g[d]));
            }
        }
    for (size_t x = 0; x < gvd.size(); x++) {
        ev = std::max(ev, std::fabs(gvd[x] - from_bf16(hgv[x])));
        mv = std::max(mv, std::fabs(gvd[x]));
        ek = std::max(ek, (double)std::fabs(from_bf16(hgk[x])));
    }
    check("attention o (q = 0: mean of the visible v)", eo / mo, 1e-2);
    check("attention lse (ln of the visible count)", el, 1e-4);
    check("attention dq (closed form)", eq / mq, 2e-2);
    check("attention dk (0 for q = 0)", ek, 0.0);
    check("attention dv (dO / count, summed)", ev / mv, 1e-2);
    for (void *p : {dq_, dk_, dv_, ddo, o, lse, gq, gk, gv, ws}) CALL(dm_device_free(p));
    return 0;
}

int decode_check() {
    const int64_t B = 3, S = 500, Hq = 8, Hkv = 2, D = 128;
    std::vector<uint16_t> q(B * Hq * D, to_bf16(0.f)), k(B * S * Hkv * D), v(B * S * Hkv * D);
    for (int64_t x = 0; x < (int64_t)k.size(); x++) {
        k[x] = to_bf16((float)(x % 13) - 6.f);
        v[x] = to_bf16((float)((x * 7) % 19) - 9.f);
    }
    const std::vector<int32_t> lens = {1, 200, 500};
    dm_attention_desc desc;
    std::memset(&desc, 0, sizeof(desc));
    desc.b = B, desc.tq = 1, desc.tk = S, desc.hq = Hq, desc.hkv = Hkv, desc.d = D;
    desc.dtype = DM_BF16, desc.mask_kind = DM_MASK_NONE;
    desc.options.window_left = desc.options.window_right = DM_UNBOUNDED;
    desc.options.deterministic = 1;
    void *dq_ = upload(q), *dk_ = upload(k), *dv_ = upload(v), *dl = upload(lens), *o = nullptr,
         *ws = nullptr;
    CALL(dm_device_alloc(q.size() * 2, &o));
    const size_t wsb = dm_attention_decode_workspace(&desc);
    CALL(dm_device_alloc(wsb, &ws));
    CALL(dm_attention_decode(&desc, dq_, dk_, dv_, (const int32_t *)dl, o, ws, wsb, nullptr));
    const auto ho = download<uint16_t>(o, q.size());
    double err = 0, mx = 0;
    for (int64_t b = 0; b < B; b++)
        for (int64_t h = 0; h < Hq; h++)
            for (int64_t d = 0; d < D; d++) {
                double s = 0;
                for (int64_t j = 0; j < lens[b]; j++)
                    s += from_bf16(v[((b * S + j) * Hkv + h / (Hq / Hkv)) * D + d]);
                s /= lens[b];
                err = std::max(err, std::fabs(s - from_bf16(ho[(b * Hq + h) * D + d])));
                mx = std::max(mx, std::fabs(s));
            }
    check("decode (q = 0: mean of the cached v)", err / mx, 1e-2);
    for (void *p : {dq_, dk_, dv_, dl, o, ws}) CALL(dm_device_free(p));
    return 0;
}

int step_check() {
    const int64_t B = 5, H = 3, Dk = 64, Dv = 96;
    const float beta_v = 0.5f, scale = 0.25f;
    std::vector<uint16_t> q(B * H * Dk), k(B * H * Dk), v(B * H * Dv);
    for (size_t x = 0; x < q.size(); x++) {
        q[x] = to_bf16((float)(x % 5) - 2.f);
        k[x] = to_bf16((float)((x * 3) % 7) - 3.f);
    }
    for (size_t x = 0; x < v.size(); x++) v[x] = to_bf16((float)((x * 5) % 11) - 5.f);
    const std::vector<float> g(B * H, -0.3f), beta(B * H, beta_v), st0(B * H * Dk * Dv, 0.f);
    dm_gdr_desc desc;
    std::memset(&desc, 0, sizeof(desc));
    desc.b = B, desc.t = 1, desc.h = H, desc.dk = Dk, desc.dv = Dv;
    desc.dtype = DM_BF16, desc.g_dtype = DM_F32, desc.beta_dtype = DM_F32;
    desc.has_scale = 1, desc.scale = scale;
    void *dq_ = upload(q), *dk_ = upload(k), *dv_ = upload(v), *dg = upload(g), *db = upload(beta),
         *ds = upload(st0), *out = nullptr;
    CALL(dm_device_alloc(v.size() * 2, &out));
    CALL(dm_gdr_step(&desc, dq_, dk_, dv_, dg, db, (const float *)ds, (float *)ds, out, nullptr));
    const auto ho = download<uint16_t>(out, v.size());
    const auto hs = download<float>(ds, st0.size());
    double eo = 0, es = 0, mo = 0;
    for (int64_t r = 0; r < B * H; r++) {
        double kq = 0;
        for (int64_t d = 0; d < Dk; d++) kq += (double)from_bf16(k[r * Dk + d]) * from_bf16(q[r * Dk + d]);
        for (int64_t c = 0; c < Dv; c++) {
            const double vc = from_bf16(v[r * Dv + c]);
            const double e = beta_v * scale * kq * vc;
            eo = std::max(eo, std::fabs(e - from_bf16(ho[r * Dv + c])));
            mo = std::max(mo, std::fabs(e));
            for (int64_t d = 0; d < Dk; d++)
                es = std::max(es, std::fabs(beta_v * from_bf16(k[r * Dk + d]) * vc -
                                            hs[(r * Dk + d) * Dv + c]));
        }
    }
    check("step out (zero state: beta scale (k . q) v)", eo / mo, 1e-2);
    check("step state (zero state: beta k v^T)", es, 1e-6);
    for (void *p : {dq_, dk_, dv_, dg, db, ds, out}) CALL(dm_device_free(p));
    return 0;
}

}  // namespace

int main() {
    char info[256];
    if (dm_describe(info, sizeof info) != DM_OK) {
        std::printf("no usable device: %s\n", dm_last_error());
        return 2;
    }
    std::printf("%s\n", info);
    if (attention_check() || decode_check() || step_check()) return 1;
    std::printf(failures ? "FAILED: %d checks\n" : "all checks passed\n", failures);
    return failures ? 1 : 0;
}
