// One LOCKS decode step driven through the plain C ABI (include/locks_hip.h)
// from C++, with no Python in the process: the way a non-Python host binds
// the library.  The host owns every buffer (hipMalloc), as the ABI requires.
//
//   summary build -> page parameters -> rki4 page scores -> GQA combine + top-b
//   -> split-K sparse decode with the merge folded in
//
// The output is checked against a host fp32 softmax attention over exactly
// the pages the selector returned; the page table's structure (sink, window,
// ascending ids, count) is checked against the derive rule.  Exit code 0 and
// a "capi ok" line on success.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "locks_hip.h"

namespace {

constexpr int R = 1, NKV = 2, G = 4, H = NKV * G, D = 128, PAGE = 16;
constexpr int SEQ = 16 * 60 + 7;                  // 61 pages, the last one partial
constexpr int MP = 64, NB = 72;
constexpr int SINK = 1, WINDOW = 1, BUDGET = 8, SPLIT = 16, PPS_MIN = 1;

uint32_t lcg = 12345u;
float urand() {                                    // deterministic, in [-1, 1)
    lcg = lcg * 1664525u + 1013904223u;
    return (float)((lcg >> 8) & 0xFFFFFF) / 8388608.f - 1.f;
}
uint16_t to_bf16(float f) {                        // round to nearest even
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float from_bf16(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

#define HIP_OK(x)                                                              \
    do {                                                                       \
        if ((x) != hipSuccess) {                                               \
            std::printf("hip error %s at line %d\n", #x, __LINE__);            \
            return 1;                                                          \
        }                                                                      \
    } while (0)
#define LOCKS_OK(x)                                                            \
    do {                                                                       \
        if ((x) != 0) {                                                        \
            std::printf("%s failed: %s\n", #x, locks_last_error());            \
            return 1;                                                          \
        }                                                                      \
    } while (0)

template <class T>
int dev_alloc(T** p, size_t n, int fill) {
    if (hipMalloc(reinterpret_cast<void**>(p), n * sizeof(T)) != hipSuccess) return 1;
    return hipMemset(*p, fill, n * sizeof(T)) != hipSuccess;
}

}  // namespace

int main() {
    if (locks_abi_version() != LOCKS_ABI_VERSION) {
        std::printf("ABI %d != %d\n", locks_abi_version(), LOCKS_ABI_VERSION);
        return 1;
    }
    // ---- host data: paged K/V cache (NB, 2, page, n_kv, d), q, block table
    const long s_tok = (long)NKV * D, s_half = (long)PAGE * s_tok, s_blk = 2 * s_half;
    std::vector<uint16_t> kv((size_t)NB * s_blk);
    for (auto& x : kv) x = to_bf16(urand());
    std::vector<uint16_t> q((size_t)R * H * D);
    for (auto& x : q) x = to_bf16(2.f * urand());
    std::vector<int32_t> bt(MP);
    for (int i = 0; i < MP; ++i) bt[i] = (i * 37 + 11) % NB;       // a permutation of 0..71
    const int32_t seq = SEQ;
    const float scale = 1.f / std::sqrt((float)D);

    // ---- device buffers (caller-owned)
    uint16_t *d_kv, *d_q, *d_vs, *d_cs, *d_mus, *d_tag, *d_out;
    uint8_t* d_v4;
    int8_t *d_c8, *d_mu8;
    int32_t *d_bt, *d_seq, *d_blocks, *d_npg, *d_nsh, *d_bfix, *d_tab, *d_cnt, *d_ctr;
    float *d_sh, *d_pmax, *d_score, *d_m, *d_l, *d_acc;
    const int chunk = locks_score_auto_chunk(R, NKV, MP);
    const int chunks = locks_score_num_chunks(MP, chunk);
    const long wsb = locks_select_workspace_bytes(R, NKV, MP);
    uint8_t* d_ws;
    if (dev_alloc(&d_kv, kv.size(), 0) || dev_alloc(&d_q, q.size(), 0) ||
        dev_alloc(&d_v4, (size_t)NB * NKV * 8 * 64, 0) || dev_alloc(&d_vs, (size_t)NB * NKV * 8, 0) ||
        dev_alloc(&d_c8, (size_t)NB * NKV * 16 * 8, 0) || dev_alloc(&d_cs, (size_t)NB * NKV * 16, 0) ||
        dev_alloc(&d_mu8, (size_t)NB * NKV * D, 0) || dev_alloc(&d_mus, (size_t)NB * NKV, 0) ||
        dev_alloc(&d_tag, (size_t)NB * NKV * 8, 0) || dev_alloc(&d_bt, MP, 0) ||
        dev_alloc(&d_seq, R, 0) || dev_alloc(&d_blocks, MP, 0) || dev_alloc(&d_npg, R, 0) ||
        dev_alloc(&d_nsh, R, 0) || dev_alloc(&d_bfix, R, 0) ||
        dev_alloc(&d_sh, (size_t)R * NKV * G * MP, 0) || dev_alloc(&d_pmax, (size_t)R * NKV * chunks * 16, 0) ||
        dev_alloc(&d_score, (size_t)R * NKV * MP, 0) || dev_alloc(&d_tab, (size_t)R * NKV * MP, 0) ||
        dev_alloc(&d_cnt, (size_t)R * NKV, 0) || dev_alloc(&d_ws, (size_t)(wsb > 256 ? wsb : 256), 0) ||
        dev_alloc(&d_m, (size_t)R * NKV * SPLIT * G, 0) || dev_alloc(&d_l, (size_t)R * NKV * SPLIT * G, 0) ||
        dev_alloc(&d_acc, (size_t)R * NKV * SPLIT * G * D, 0) || dev_alloc(&d_ctr, (size_t)R * NKV * LOCKS_DECODE_COUNTER_STRIDE, 0) ||
        dev_alloc(&d_out, (size_t)R * H * D, 0)) {
        std::printf("allocation failed\n");
        return 1;
    }
    HIP_OK(hipMemcpy(d_kv, kv.data(), kv.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_q, q.data(), q.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_bt, bt.data(), MP * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_seq, &seq, 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_blocks, bt.data(), MP * 4, hipMemcpyHostToDevice));
    hipStream_t stream;
    HIP_OK(hipStreamCreate(&stream));

    // ---- summaries of the finalized pages (settled tokens: SEQ - 1)
    const int n_fin = (SEQ - 1) / PAGE;
    LOCKS_OK(locks_build_rki4(d_kv, s_blk, s_tok, D, NB, d_blocks, n_fin, NKV, D, PAGE, d_v4,
                              d_vs, d_c8, d_cs, d_mu8, d_mus, nullptr, d_tag, stream));
    LOCKS_OK(locks_derive_params(d_seq, R, PAGE, WINDOW, SINK, BUDGET, 0.1, d_npg, d_nsh, d_bfix,
                                 stream));
    LOCKS_OK(locks_score_rki4(d_q, (long)H * D, D, d_v4, d_vs, d_c8, d_cs, d_mu8, d_mus, nullptr, NB, d_bt,
                              MP, MP, d_nsh, d_sh, MP, d_pmax, chunk, R, NKV, G, D, PAGE, scale,
                              stream));
    LOCKS_OK(locks_select_nrm_topb(d_sh, d_pmax, chunks, d_npg, d_nsh, d_bfix, d_score, d_tab,
                                   d_cnt, d_ws, wsb, R, NKV, G, SINK, MP, 0, BUDGET, stream));
    LOCKS_OK(locks_decode_fused(d_q, (long)H * D, D, d_kv, s_blk, s_tok, D, d_kv + s_half, s_blk,
                                s_tok, D, NB, d_bt, MP, MP, d_tab, (long)NKV * MP, MP, MP, d_cnt,
                                NKV, d_seq, d_m, d_l, d_acc, d_ctr, d_out, (long)H * D, D, 0, R,
                                NKV, G, D, PAGE, SPLIT, PPS_MIN, BUDGET + SINK + WINDOW, scale,
                                stream));
    HIP_OK(hipStreamSynchronize(stream));

    std::vector<int32_t> tab((size_t)NKV * MP), cnt(NKV);
    std::vector<uint16_t> out((size_t)H * D);
    HIP_OK(hipMemcpy(tab.data(), d_tab, tab.size() * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(cnt.data(), d_cnt, NKV * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(out.data(), d_out, out.size() * 2, hipMemcpyDeviceToHost));

    // ---- checks
    const int npg = (SEQ + PAGE - 1) / PAGE;
    const int want_cnt = SINK + BUDGET + WINDOW;       // sink + top-b middle + recent window
    double worst = 0.0;
    for (int kh = 0; kh < NKV; ++kh) {
        const int32_t* t = &tab[(size_t)kh * MP];
        if (cnt[kh] != want_cnt) { std::printf("kv head %d: count %d != %d\n", kh, cnt[kh], want_cnt); return 1; }
        if (t[0] != 0 || t[cnt[kh] - 1] != npg - 1) { std::printf("kv head %d: sink/window missing\n", kh); return 1; }
        for (int i = 1; i < cnt[kh]; ++i)
            if (t[i] <= t[i - 1]) { std::printf("kv head %d: page ids not ascending\n", kh); return 1; }
        for (int g = 0; g < G; ++g) {
            const int h = kh * G + g;
            std::vector<double> s, o(D, 0.0);
            std::vector<long> rows;
            for (int i = 0; i < cnt[kh]; ++i)
                for (int tk = 0; tk < PAGE; ++tk) {
                    const int pos = t[i] * PAGE + tk;
                    if (pos >= SEQ) continue;
                    const long base = (long)bt[t[i]] * s_blk + tk * s_tok + kh * D;
                    double dot = 0.0;
                    for (int e = 0; e < D; ++e) dot += (double)from_bf16(q[h * D + e]) * from_bf16(kv[base + e]);
                    s.push_back(dot * scale);
                    rows.push_back(base + s_half);
                }
            double mx = -1e300, den = 0.0;
            for (double x : s) mx = x > mx ? x : mx;
            for (size_t j = 0; j < s.size(); ++j) {
                const double p = std::exp(s[j] - mx);
                den += p;
                for (int e = 0; e < D; ++e) o[e] += p * from_bf16(kv[rows[j] + e]);
            }
            for (int e = 0; e < D; ++e) {
                const double err = std::fabs(o[e] / den - from_bf16(out[h * D + e]));
                worst = err > worst ? err : worst;
            }
        }
    }
    if (!(worst <= 2e-2)) { std::printf("decode mismatch: max|d| = %.3e\n", worst); return 1; }
    std::printf("capi ok: %d pages per kv head, decode max|d| = %.3e\n", cnt[0], worst);
    return 0;
}
