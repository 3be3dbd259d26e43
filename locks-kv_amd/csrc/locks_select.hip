// GQA combine + exact top-b page selection for gfx950, and the per-step
// page-parameter derivation.
//
// Semantics (reference: selection/select_cuda.py:547-828 fused nrm+top-b,
// selection/select.py:28-58 derive, selection/select.py:123-180 top-b twin):
//   hm[g]    = max_{0<=p<nsh} score_h[g][p]                    ("nrm" only)
//   score[p] = sum_{g ascending} exp(score_h[g][p] - hm[g])    ("nrm")
//            = max_g score_h[g][p]                             ("max")
//   keep     = top-b of the selectable slice [sink, nsh) under the total
//              order (score descending, page ascending) -- i.e. every page
//              above the b-th largest score tau plus the lowest-index pages
//              equal to tau up to exactly b -- U [0, sink) U [nsh, npg);
//              (nsh - sink) <= 1 keeps every page of [0, npg).
//   page_table[r][kh][:cnt] = kept pages ascending, -1 after; page_cnt = cnt.
//
// MI355X design.  At 1M context one (request, kv head) has 65536 pages and
// bs=1 GLM has only two such groups, so a one-workgroup-per-group selector
// would read 4 MB of score_h through a single CU.  Instead:
//   sel_chunk_kernel  (grid: page chunks x kv heads x requests)
//       forms hm from the scorer's per-chunk maxima, combines its 2048-page
//       chunk, writes `score`, prefills its slice of page_table with -1, and
//       emits the chunk's local top-b candidates (the total order restricted
//       to a chunk keeps every globally kept page of that chunk) in ascending
//       page order.  When one chunk covers the whole row it finishes the
//       selection itself (one launch).
//   sel_finish_kernel (grid: kv heads x requests)
//       gathers the <= b candidates of every chunk into LDS, radix-selects
//       the exact b-th largest key and compacts the kept pages.
// (Folding the finish into the last-arriving chunk needs an agent-scope
// release fence, which on MI355X writes back the XCD's dirty L2 and measured
// slower than the second launch.)
// Radix keys are the order-preserving fp32 -> u32 map; the keep test is a
// key compare, so it is exact for every finite score.
#include <type_traits>

#include "locks_common.h"
#include "locks_hip.h"

namespace locks {

constexpr int SEL_CH = 2048;       // pages per chunk workgroup
constexpr int SEL_BLK = 512;       // threads per chunk workgroup
constexpr int FIN_BLK = 1024;      // threads of the finishing workgroup
constexpr int FIN_CAP = 6144;      // candidates held in LDS by the finisher
constexpr int FIN_MAXZ = 1024;     // chunks per row the finisher can index

// ---------------------------------------------------------------------------
// block primitives
// ---------------------------------------------------------------------------
// TAIL: the closing barrier that lets the caller reuse wsum right away
template <int BLK, bool TAIL = true>
__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int& total) {
    constexpr int NW = BLK / kWave;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int incl = wave_incl_scan_i(v);
    if (lane == kWave - 1) wsum[w] = incl;
    lds_barrier();
    if (w == 0) {
        const int x = (lane < NW) ? wsum[lane] : 0;
        const int xi = wave_incl_scan_i(x);
        if (lane < NW) wsum[lane] = xi - x;
        if (lane == NW - 1) wsum[NW] = xi;
    }
    lds_barrier();
    const int res = wsum[w] + incl - v;
    total = wsum[NW];
    if constexpr (TAIL) lds_barrier();
    return res;
}

// LDS histogram increment with wave aggregation: lanes whose bin equals the
// first active lane's bin are counted by one atomic (scores cluster, so most
// keys of a digit pass share a bin and plain LDS atomics serialize).
__device__ __forceinline__ void hist_add(int* hist, int bin, bool valid) {
    const int lane = threadIdx.x & 63;
    const unsigned long long act = __ballot(valid);
    if (act == 0ull) return;
    const int leader = __ffsll((long long)act) - 1;       // wave-uniform
    const int b0 = __builtin_amdgcn_readlane(bin, leader);
    const bool same = valid && bin == b0;
    const unsigned long long m = __ballot(same);
    if (lane == leader) atomicAdd(&hist[b0], __popcll(m));
    if (valid && !same) atomicAdd(&hist[bin], 1);
}

// k-th largest (1 <= k <= n) u32 key by 4 passes of 8-bit MSD radix.  If a
// pass finds that the whole boundary bin is needed it stops early and the
// returned value has zero low digits (then #(key >= result) == k exactly).
template <int BLK>
__device__ uint32_t block_kth_largest(const uint32_t* keys, int n, int k, int* hist, int* s3) {
    const int tid = threadIdx.x;
    uint32_t prefix = 0u, kmask = 0u;
    for (int digit = 0; digit < 4; ++digit) {
        const int shift = 24 - 8 * digit;
        for (int i = tid; i < 256; i += BLK) hist[i] = 0;
        lds_barrier();
        // 16 keys per thread in flight per batch (keys may live in global
        // memory: a key-at-a-time loop would serialize one latency per key)
        for (int i0 = tid; i0 < n; i0 += 16 * BLK) {
            uint32_t u[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int i = i0 + j * BLK;
                u[j] = (i < n) ? keys[i] : 0u;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j)
                hist_add(hist, (u[j] >> shift) & 0xFF, (i0 + j * BLK < n) && (u[j] & kmask) == prefix);
        }
        lds_barrier();
        if (tid < kWave) {
            const int lane = tid;
            const int seg = hist[4 * lane] + hist[4 * lane + 1] + hist[4 * lane + 2] + hist[4 * lane + 3];
            int suf = seg;
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const int t = __shfl_down(suf, o, kWave);
                if (lane + o < kWave) suf += t;
            }
            const int above = suf - seg;
            if (above < k && k <= suf) {
                int acc = above, sel = 4 * lane, cb = 0;
                for (int d = 4 * lane + 3; d >= 4 * lane; --d) {
                    const int c = hist[d];
                    if (acc + c >= k) { sel = d; cb = c; break; }
                    acc += c;
                }
                s3[0] = sel;
                s3[1] = k - acc;
                s3[2] = cb;
            }
        }
        lds_barrier();
        prefix |= ((uint32_t)s3[0]) << shift;
        k = s3[1];
        const int cb = s3[2];
        kmask |= 0xFFu << shift;
        lds_barrier();
        if (k == cb) break;
    }
    return prefix;
}

// Ordered emission of the top-k of keys[0, n) (page order) under
// (key descending, index ascending): every key > tau plus the first
// (k - #(>tau)) keys == tau.  Writes out_page[pos] = page_of(i) and, if
// out_key != nullptr, out_key[pos] = key.  Returns the count (== k).
template <int BLK, class PageOf>
__device__ int emit_topk(const uint32_t* keys, int n, int k, uint32_t tau, PageOf page_of,
                         int* out_page, uint32_t* out_key, int* wsum) {
    const int tid = threadIdx.x;
    const int E = cdiv(n, BLK);
    const int i0 = min(tid * E, n), i1 = min(i0 + E, n);
    int gt = 0, eq = 0;
    for (int b0 = i0; b0 < i1; b0 += 16) {              // 16 loads in flight
        uint32_t u[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) u[j] = (b0 + j < i1) ? keys[b0 + j] : 0u;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            gt += (b0 + j < i1) && (u[j] > tau);
            eq += (b0 + j < i1) && (u[j] == tau);
        }
    }
    int gt_tot, eq_tot;
    block_excl_scan<BLK>(gt, wsum, gt_tot);
    const int eq_excl = block_excl_scan<BLK>(eq, wsum, eq_tot);
    const int quota = k - gt_tot;
    const int mine = gt + min(max(quota - eq_excl, 0), eq);
    int total;
    int pos = block_excl_scan<BLK>(mine, wsum, total);
    int er = eq_excl;
    for (int b0 = i0; b0 < i1; b0 += 16) {
        uint32_t u[16];
        int pg[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            u[j] = (b0 + j < i1) ? keys[b0 + j] : 0u;
            pg[j] = (b0 + j < i1) ? page_of(b0 + j) : 0;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const bool in = b0 + j < i1;
            bool kp = in && u[j] > tau;
            if (in && u[j] == tau) { kp = er < quota; ++er; }
            if (kp) {
                out_page[pos] = pg[j];
                if (out_key) out_key[pos] = u[j];
                ++pos;
            }
        }
    }
    return total;
}

// Max over one head's n per-chunk maxima p[0 .. n) (the scorer's page_max
// is head-major, so a wave's loads are contiguous), 4 independent loads in
// flight per lane (a serial load chain costs one memory latency per step).
__device__ __forceinline__ float chunk_max(const float* __restrict__ p, int n) {
    const int lane = threadIdx.x & 63;
    float m = -INFINITY;
    for (int z0 = lane; z0 < n; z0 += 4 * kWave) {
        float t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)                    // clamped: a repeat leaves the max
            t[j] = p[min(z0 + j * kWave, n - 1)];
#pragma unroll
        for (int j = 0; j < 4; ++j) m = fmaxf(m, t[j]);
    }
    return m;
}

__device__ __forceinline__ void fill_all_pages(int* row, int n_pages, int MP, bool pad) {
    for (int i = threadIdx.x; i < MP; i += blockDim.x) {
        if (i < n_pages) row[i] = i;
        else if (pad) row[i] = -1;
    }
}

// Finish one row from the chunk candidates (ascending page order per chunk):
// exact b-th largest key over all candidates, ordered emission, sink/window.
// LDS arguments: offs[FIN_MAXZ+1], lkey/lpage[cap] (more candidates spill to
// the global workspace), hist[256], s3[4], wsum.
template <int BLK>
__device__ void finish_row(long rk, int n_pages, int n_sel_hi, int n_sink, int b, int MP, int Z1,
                           int* __restrict__ trow, int* __restrict__ cnt_out,
                           const uint32_t* __restrict__ cand_key, const int* __restrict__ cand_page,
                           const int* __restrict__ cand_cnt, uint32_t* __restrict__ spill_key,
                           int* __restrict__ spill_page, int* offs, uint32_t* lkey, int* lpage,
                           int* hist, int* s3, int* wsum, int cap = FIN_CAP) {
    constexpr int NWV = BLK / kWave;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    {
        int run = 0;
        for (int base = 0; base < Z1; base += BLK) {
            const int zz = base + tid;
            const int c = (zz < Z1) ? cand_cnt[rk * Z1 + zz] : 0;
            int tot;
            const int ex = block_excl_scan<BLK>(c, wsum, tot);
            if (zz < Z1) offs[zz] = run + ex;
            run += tot;
        }
        if (tid == 0) offs[Z1] = run;
        lds_barrier();
    }
    const int N = offs[Z1];
    uint32_t* kk = (N <= cap) ? lkey : spill_key + rk * (long)MP;
    int* pp = (N <= cap) ? lpage : spill_page + rk * (long)MP;
    for (int zz = wave; zz < Z1; zz += NWV) {                 // chunk order == page order
        const int o = offs[zz], c = offs[zz + 1] - o;
        const uint32_t* sk = cand_key + (rk * Z1 + zz) * (long)SEL_CH;
        const int* sp = cand_page + (rk * Z1 + zz) * (long)SEL_CH;
        for (int i0 = lane; i0 < c; i0 += 8 * kWave) {      // 8 loads in flight
            uint32_t kv[8];
            int pv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * kWave;
                kv[j] = (i < c) ? sk[i] : 0u;
                pv[j] = (i < c) ? sp[i] : 0;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * kWave;
                if (i < c) { kk[o + i] = kv[j]; pp[o + i] = pv[j]; }
            }
        }
    }
    __syncthreads();                    // candidates may be in global spill memory
    const uint32_t tau = block_kth_largest<BLK>(kk, N, b, hist, s3);
    const int nsel_w = emit_topk<BLK>(kk, N, b, tau, [&](int i) { return pp[i]; },
                                      trow + n_sink, nullptr, wsum);
    const int cnt = n_sink + nsel_w + (n_pages - n_sel_hi);
    for (int i = tid; i < n_sink; i += BLK) trow[i] = i;
    for (int i = n_sink + nsel_w + tid; i < cnt; i += BLK) trow[i] = n_sel_hi + (i - n_sink - nsel_w);
    if (tid == 0) *cnt_out = cnt;
}

// ---------------------------------------------------------------------------
// register-resident exact top-k: thread t holds keys[E] (valid flags) of
// consecutive items.  Result: either a whole bin (every key >= lo is kept)
// or an exact threshold (keys > tau kept, then keys == tau up to k).
// Items must number < 65536.
// ---------------------------------------------------------------------------
struct RadixSel {
    uint32_t lo, tau;
    int k;              // keys == tau still to take (exact mode)
    bool whole_bin;     // every key >= lo is kept
};

// Boundary search over an LDS histogram of nb bins (nb = 4096 or 256): the
// bin B holding the k-th largest (bins counted from the top), the keys still
// needed from it (k - #above) and its count, in s3[0..2].
template <int BLK, int NB>
__device__ __forceinline__ void hist_boundary(const int* hist, int k, int* wtot, int* s3) {
    constexpr int NW = BLK / kWave;
    constexpr int nb = NB;
    constexpr int bpl = NB / BLK > 0 ? NB / BLK : 1;    // histogram bins per lane
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // thread t: bins top .. top-bpl+1, top = nb-1-bpl*t (ascending thread
    // order = descending bin order)
    const int top = nb - 1 - bpl * tid;
    int c = 0;
#pragma unroll
    for (int j = 0; j < bpl; ++j) c += (top - j >= 0) ? hist[top - j] : 0;
    const int incl = wave_incl_scan_i(c);
    if (lane == kWave - 1) wtot[wave] = incl;
    lds_barrier();
    // counts of the waves before this one: one parallel LDS read and a
    // wave sum (a serial loop would chain up to NW - 1 LDS latencies)
    const int base = wave_sum_i((lane < wave && lane < NW) ? wtot[lane] : 0);
    const int above0 = base + incl - c;
    if (c > 0 && above0 < k && k <= base + incl) {
        int above = above0;
#pragma unroll
        for (int j = 0; j < bpl; ++j) {
            const int cb = (top - j >= 0) ? hist[top - j] : 0;
            if (above + cb >= k) { s3[0] = top - j; s3[1] = k - above; s3[2] = cb; break; }
            above += cb;
        }
    }
    lds_barrier();
}

// 12 + 12 + 8-bit MSD radix on the absolute key bits (the fallback of
// reg_kth_largest below).
template <int BLK, int E>
__device__ RadixSel reg_kth_largest_abs(const uint32_t (&key)[E], const bool (&val)[E], int k,
                                        int* hist, int* wtot, int* s3) {
    const int tid = threadIdx.x;
    uint32_t prefix = 0u, kmask = 0u;
#pragma unroll 1
    for (int pass = 0; pass < 3; ++pass) {
        const int shift = pass == 0 ? 20 : pass == 1 ? 8 : 0;
        const int nb = pass < 2 ? 4096 : 256;
        for (int i = tid; i < nb; i += BLK) hist[i] = 0;
        lds_barrier();
#pragma unroll
        for (int e = 0; e < E; ++e)
            hist_add(hist, (int)((key[e] >> shift) & (uint32_t)(nb - 1)),
                     val[e] && (key[e] & kmask) == prefix);
        lds_barrier();
        if (pass < 2) hist_boundary<BLK, 4096>(hist, k, wtot, s3);
        else hist_boundary<BLK, 256>(hist, k, wtot, s3);
        prefix |= ((uint32_t)s3[0]) << shift;
        kmask |= ((uint32_t)(nb - 1)) << shift;
        const int cb = s3[2];
        k = s3[1];
        if (k == cb) return RadixSel{prefix, prefix, k, true};   // keys >= prefix (low bits 0)
    }
    return RadixSel{prefix, prefix, k, false};
}

// Exact k-th largest with a first pass relative to the row maximum mk: bin
// = 4095 - min(4095, (mk - key) >> 15), i.e. 4096 bins of 2^15 key steps
// (about 2^-8 of a binade) covering the 16 binades below the maximum, keys
// further down clamped into bin 0.  The top keys spread over many bins
// instead of the few that the absolute leading bits give, so the boundary
// bin usually holds the last needed key alone and the select ends after
// one pass; otherwise a second pass splits the 2^15-step bin into 4096 bins
// of 8 steps and a third pass resolves the 8 -- or, with COMPACT, a
// boundary bin of at most 64 keys is gathered into LDS and ranked by one wave
// (two barriers instead of two histogram passes: row select -1.5 us at
// Llama 128K, chunk select -0.7 us at 1M).  A boundary in the clamped bin 0
// (the k-th key more than 16 binades below the maximum) falls back to the
// absolute radix.
//
// mk_bound != 0: an upper bound of every valid key known to the caller (the
// bins are placed relative to it instead of the exact maximum, one block
// reduction and barrier fewer); the caller has then also zeroed hist and
// s3[3] before a barrier that every thread passed since.
template <int BLK, int E, bool COMPACT = true>
__device__ RadixSel reg_kth_largest(const uint32_t (&key)[E], const bool (&val)[E], int k,
                                    int* hist, int* wtot, int* s3, uint32_t mk_bound = 0u) {
    constexpr int NW = BLK / kWave;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint32_t mk = mk_bound;
    if (mk_bound == 0u) {
        // row maximum over the valid keys (0 when none: every valid key >= 0)
        uint32_t mx = 0u;
#pragma unroll
        for (int e = 0; e < E; ++e) mx = val[e] ? max(mx, key[e]) : mx;
        for (int i = tid; i < 4096; i += BLK) hist[i] = 0;
        if (tid == 0) s3[3] = 0;                              // candidate counter (compaction below)
        mx = wave_max_u32(mx);
        if (lane == 0) wtot[wave] = (int)mx;
        lds_barrier();
#pragma unroll
        for (int w = 0; w < NW; ++w) mk = max(mk, (uint32_t)wtot[w]);
    }
    // pass 0: bins relative to mk.  One LDS atomic per key (the keys of a
    // wave mostly fall into distinct bins here, and the wave-aggregated
    // add's ballot / lane-read chain cost more than it saved: Llama 128K
    // row select 9.05 -> 8.17 us); keys clamped into bin 0 (more than 16
    // binades below mk, often most of a row) are counted in registers and
    // added once per wave instead of contending for one address.
    {
        int nclamp = 0;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const uint32_t d = (mk - key[e]) >> 15;
            if (val[e] && d < 4095u) atomicAdd(&hist[4095 - (int)d], 1);
            nclamp += (val[e] && d >= 4095u) ? 1 : 0;
        }
        nclamp = wave_sum_i(nclamp);
        if (lane == 0 && nclamp > 0) atomicAdd(&hist[0], nclamp);
    }
    lds_barrier();
    hist_boundary<BLK, 4096>(hist, k, wtot, s3);
    const int B = s3[0];
    if (B == 0) return reg_kth_largest_abs<BLK, E>(key, val, k, hist, wtot, s3);
    // bin B holds keys with (mk - key) >> 15 == 4095 - B: [lo, hi] (a
    // non-empty bin implies mk >= (4095 - B) << 15, so hi does not wrap;
    // lo saturates at 0)
    const uint32_t span = (uint32_t)(4096 - B) << 15;
    uint32_t hi = mk - ((uint32_t)(4095 - B) << 15);
    uint32_t lo = (mk + 1u > span) ? mk + 1u - span : 0u;
    k = s3[1];
    const int cb = s3[2];
    if (k == cb) return RadixSel{lo, lo, k, true};
    if (COMPACT && cb <= kWave) {
        // Few keys in the boundary bin: gather them into LDS and let one
        // wave rank them with lane reads, instead of two more histogram
        // passes over every key.
        int* cand = hist;                                     // the histogram is consumed
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (val[e] && key[e] >= lo && key[e] <= hi) cand[atomicAdd(&s3[3], 1)] = (int)key[e];
        lds_barrier();
        if (wave == 0) {
            const uint32_t c = lane < cb ? (uint32_t)cand[lane] : 0u;
            int gt = 0, eqb = 0;                              // descending rank of this lane's key
            for (int j = 0; j < cb; ++j) {
                const uint32_t cj = (uint32_t)__builtin_amdgcn_readlane((int)c, j);
                gt += cj > c;
                eqb += (cj == c) & (j < lane);
            }
            const unsigned long long at = __ballot(lane < cb && gt + eqb == k - 1);
            const uint32_t tau = (uint32_t)__builtin_amdgcn_readlane((int)c, __ffsll((long long)at) - 1);
            const int above = __popcll(__ballot(lane < cb && c > tau));
            if (lane == 0) { s3[0] = (int)tau; s3[1] = k - above; }
        }
        lds_barrier();
        const uint32_t tau = (uint32_t)s3[0];
        return RadixSel{tau, tau, s3[1], false};              // keys > tau, then s3[1] keys == tau
    }
    // passes 1 and 2: bins of 8 steps inside [lo, hi] (< 2^15 steps), then
    // the (<= 8) steps of the boundary bin
#pragma unroll 1
    for (int pass = 1; pass < 3; ++pass) {
        const int shift = pass == 1 ? 3 : 0;
        const int nb = pass == 1 ? 4096 : 8;
        for (int i = tid; i < nb; i += BLK) hist[i] = 0;
        lds_barrier();
#pragma unroll
        for (int e = 0; e < E; ++e)
            hist_add(hist, (int)((key[e] - lo) >> shift) & (nb - 1), val[e] && key[e] >= lo && key[e] <= hi);
        lds_barrier();
        if (pass == 1) hist_boundary<BLK, 4096>(hist, k, wtot, s3);
        else hist_boundary<BLK, 8>(hist, k, wtot, s3);
        lo += (uint32_t)s3[0] << shift;
        hi = min(hi, lo + ((1u << shift) - 1u));
        const int cb = s3[2];
        k = s3[1];
        if (k == cb) return RadixSel{lo, lo, k, true};
    }
    return RadixSel{lo, lo, k, false};                        // exact: tau = lo
}

// Emission in item order: out(pos, e) is called for every kept item of
// this thread with its rank among all kept items.  Returns the kept count.
template <int BLK, int E, bool TAIL = true, class Out>
__device__ int reg_emit(const uint32_t (&key)[E], const bool (&val)[E], const RadixSel& rs,
                        int* wsum, Out out) {
    int gt = 0, eq = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if (!val[e]) continue;
        if (rs.whole_bin) gt += key[e] >= rs.lo;
        else { gt += key[e] > rs.tau; eq += key[e] == rs.tau; }
    }
    int tot;
    const int ex = block_excl_scan<BLK, TAIL>(gt | (eq << 16), wsum, tot);
    const int quota = rs.whole_bin ? 0 : rs.k;
    int pos = (ex & 0xFFFF) + min(ex >> 16, quota);
    int er = ex >> 16;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        if (!val[e]) continue;
        bool kp;
        if (rs.whole_bin) kp = key[e] >= rs.lo;
        else {
            kp = key[e] > rs.tau;
            if (key[e] == rs.tau) { kp = er < quota; ++er; }
        }
        if (kp) out(pos++, e);
    }
    return (tot & 0xFFFF) + min(tot >> 16, quota);
}

// ---------------------------------------------------------------------------
// whole-row kernel (max_pages <= ROW_MAXP): one 1024-thread workgroup per
// (request, kv head) does combine, exact top-b and the page table in one
// launch.  Thread t owns pages [E t, E t + E) (contiguous, so one packed
// block scan orders the emission); the keys stay in registers; the radix
// select runs 12 + 12 + 8-bit MSD passes over an LDS histogram.
// ---------------------------------------------------------------------------
constexpr int ROW_BLK = 1024;
constexpr int ROW_NW = ROW_BLK / kWave;
// Above 8192 pages a row's score_h (G x pages x 4 B) through one CU is
// slower than the page-parallel route (measured: 16384 pages, G = 4: 22.4 vs
// 20.5 us; G = 16: 44.8 vs 25.7 us).
constexpr int ROW_MAXP = 8 * ROW_BLK;

template <int E, int HB = (E <= 8) ? 8 : 4>
__global__ __launch_bounds__(ROW_BLK) void sel_row_kernel(
    const float* __restrict__ score_h, const float* __restrict__ pmax, int Zs,
    const int* __restrict__ npg, const int* __restrict__ nsh, const int* __restrict__ bfix,
    float* __restrict__ score, int* __restrict__ page_table, int* __restrict__ page_cnt,
    int n_sink, int MP, int G, int combine)
{
    static_assert(E % 4 == 0, "pages per thread must be a multiple of 4");
    const int kh = blockIdx.x, r = blockIdx.y, n_kv = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long rk = (long)r * n_kv + kh;
    const int n_pages = max(min(npg[r], MP), 0);
    const int n_sel_hi = min(nsh[r], MP);
    const int n_sel = n_sel_hi - n_sink;
    const bool keep_all = n_sel <= 1;
    int b = bfix[r];
    b = max(1, min(b, max(n_sel, 1)));
    const int pend = max(n_sel_hi, 0);                    // score written for p < pend
    const int p0 = tid * E;

    __shared__ float hm[16];
    __shared__ int hist[4096];
    __shared__ int wtot[ROW_NW];
    __shared__ int s3[4];
    __shared__ int wsum[ROW_NW + 1];
    // nrm: the radix histogram is zeroed here, ahead of the head-max barrier
    // (the selection then needs no barrier of its own before its first pass)
    if (combine == 0) {
        for (int i = tid; i < 4096; i += ROW_BLK) hist[i] = 0;
        if (tid == 0) s3[3] = 0;
    }

    // ---- score_h of the first HB heads in flight before the head maxima.
    // Loads are bounded by the row (MP), not by n_sel_hi, so they do not wait
    // for the per-request parameters; pages >= n_sel_hi are ignored below.
    // HB heads per load batch: the host passes 4 for groups of at most 4
    // (the clamped loads of heads past G re-read the last head)
    const float* shb = score_h + rk * (long)G * MP;
    float4 xv[HB][E / 4];
    auto load_batch = [&](int g0) {
#pragma unroll
        for (int j = 0; j < HB; ++j)
#pragma unroll
            for (int v = 0; v < E / 4; ++v) {
                // unconditional (clamped) loads: surplus heads / pages are
                // never combined or kept, and a guarded load would make the
                // compiler wait for it before the page maxima are requested
                const int g = min(g0 + j, G - 1), p = min(p0 + 4 * v, MP - 4);
                xv[j][v] = *reinterpret_cast<const float4*>(shb + (long)g * MP + p);
            }
    };
    load_batch(0);
    if (combine == 0) {
        if (wave < G) {
            float m = -INFINITY;
            m = chunk_max(pmax + (rk * 16 + wave) * Zs, Zs);
            m = wave_max(m);
            if (lane == 0) hm[wave] = m;
        }
        lds_barrier();
    }
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = (combine == 0) ? 0.f : -INFINITY;
    // The combine mode is tested once, outside the loops, and heads past G
    // are masked by selects, not branches: a uniform branch per element
    // split every exp into its own basic block (no overlap between them).
    // Heads are summed in ascending order either way.
    for (int g0 = 0; g0 < G; g0 += HB) {
        if (g0 > 0) load_batch(g0);
        if (combine == 0) {
#pragma unroll
            for (int j = 0; j < HB; ++j) {
                const bool on = g0 + j < G;
                const float h = hm[min(g0 + j, G - 1)];
#pragma unroll
                for (int v = 0; v < E / 4; ++v) {
                    const float x4[4] = {xv[j][v].x, xv[j][v].y, xv[j][v].z, xv[j][v].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float t = __expf(x4[i] - h);
                        acc[4 * v + i] = on ? acc[4 * v + i] + t : acc[4 * v + i];
                    }
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < HB; ++j) {
                const int g = g0 + j;
#pragma unroll
                for (int v = 0; v < E / 4; ++v) {
                    const float x4[4] = {xv[j][v].x, xv[j][v].y, xv[j][v].z, xv[j][v].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float mx = (g == 0) ? x4[i] : fmaxf(acc[4 * v + i], x4[i]);
                        acc[4 * v + i] = (g < G) ? mx : acc[4 * v + i];
                    }
                }
            }
        }
    }
    float* srow = score + rk * (long)MP;
    if (p0 + E <= pend) {
#pragma unroll
        for (int v = 0; v < E / 4; ++v)
            *reinterpret_cast<float4*>(srow + p0 + 4 * v) = make_float4(acc[4 * v], acc[4 * v + 1], acc[4 * v + 2], acc[4 * v + 3]);
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e)
            if (p0 + e < pend) srow[p0 + e] = acc[e];
    }

    int* trow = page_table + rk * (long)MP;
    if (keep_all || b >= n_sel) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int i = p0 + e;
            if (i < MP) trow[i] = (i < n_pages) ? i : -1;
        }
        if (tid == 0) page_cnt[rk] = n_pages;
        return;
    }
    // Entries that do not depend on the selection -- the sink pages, the
    // unselectable tail [nsh, npg) after the b kept pages, and the -1
    // padding -- are stored before the select, so their stores drain under
    // it instead of ahead of the kernel's end (Llama 128K row: -0.5 us)
    const int cnt = n_sink + b + (n_pages - n_sel_hi);
    if (p0 >= cnt && p0 + E <= MP) {                      // padding only
#pragma unroll
        for (int v = 0; v < E / 4; ++v) *reinterpret_cast<int4*>(trow + p0 + 4 * v) = make_int4(-1, -1, -1, -1);
    } else if (p0 < n_sink || p0 + E > n_sink + b) {     // not only kept slots
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int i = p0 + e;
            if (i >= MP) break;
            if (i < n_sink) trow[i] = i;
            else if (i >= n_sink + b && i < cnt) trow[i] = n_sel_hi + (i - n_sink - b);
            else if (i >= cnt) trow[i] = -1;
        }
    }
    if (tid == 0) page_cnt[rk] = cnt;

    // ---- exact b-th largest key among the selectable pages [n_sink, nsh) --
    uint32_t key[E];
    bool val[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int p = p0 + e;
        val[e] = (p >= n_sink) && (p < n_sel_hi);
        key[e] = f2u(acc[e]);
    }
    // nrm keys are sums of G terms exp(s - max_p s) <= 1: 2G bounds them
    // (with a binade to spare), so the bins need no block maximum
    const uint32_t mk_bound = (combine == 0) ? f2u(2.f * (float)G) : 0u;
    const RadixSel rs = reg_kth_largest<ROW_BLK, E>(key, val, b, hist, wtot, s3, mk_bound);
    // wsum is not used again: no closing barrier after the emission scan
    reg_emit<ROW_BLK, E, false>(key, val, rs, wsum, [&](int pos, int e) { trow[n_sink + pos] = p0 + e; });
}

// ---------------------------------------------------------------------------
// chunk kernel
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(SEL_BLK) void sel_chunk_kernel(
    const float* __restrict__ score_h, const float* __restrict__ pmax, int Zs,
    const int* __restrict__ npg, const int* __restrict__ nsh, const int* __restrict__ bfix,
    float* __restrict__ score, int* __restrict__ page_table, int* __restrict__ page_cnt,
    uint32_t* __restrict__ cand_key, int* __restrict__ cand_page, int* __restrict__ cand_cnt,
    int n_sink, int MP, int G, int combine)
{
    const int z = blockIdx.x, kh = blockIdx.y, r = blockIdx.z;
    const int n_kv = gridDim.y, Z1 = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long rk = (long)r * n_kv + kh;
    const int n_pages = min(npg[r], MP);
    const int n_sel_hi = min(nsh[r], MP);
    const int n_sel = n_sel_hi - n_sink;
    const bool keep_all = n_sel <= 1;
    int b = bfix[r];
    b = max(1, min(b, max(n_sel, 1)));
    const bool final_mode = (Z1 == 1);
    const int c0 = z * SEL_CH;
    const int c1 = min(c0 + SEL_CH, MP);

    __shared__ float hm[16];
    __shared__ uint32_t keys[SEL_CH];
    __shared__ int hist[256];
    __shared__ int s3[4];
    __shared__ int wsum[SEL_BLK / kWave + 1];

    int* trow = page_table + rk * (long)MP;
    if (!final_mode) {
        for (int i = c0 + tid; i < c1; i += SEL_BLK) trow[i] = -1;
    }

    // ---- issue every score_h load of this thread first (4 pages x G rows)
    const float* shb = score_h + rk * (long)G * MP;
    const int pend = min(c1, max(n_sel_hi, c0));
    constexpr int SEL_E = SEL_CH / SEL_BLK;
    float x[SEL_E][16];
#pragma unroll
    for (int e = 0; e < SEL_E; ++e) {
        const int p = c0 + tid + e * SEL_BLK;
#pragma unroll
        for (int g = 0; g < 16; ++g)
            x[e][g] = (g < G && p < pend) ? shb[(long)g * MP + p] : 0.f;
    }

    // ---- per-head page max from the scorer's chunk maxima ("nrm") --------
    if (combine == 0) {
        for (int g = wave; g < G; g += SEL_BLK / kWave) {
            float m = -INFINITY;
            m = chunk_max(pmax + (rk * 16 + g) * Zs, Zs);
            m = wave_max(m);
            if (lane == 0) hm[g] = m;
        }
        lds_barrier();
    }

    // ---- combine: score[p] for p < nsh, keys for the selectable slice ----
#pragma unroll
    for (int e = 0; e < SEL_E; ++e) {
        const int p = c0 + tid + e * SEL_BLK;
        if (p >= pend) continue;
        float acc;
        if (combine == 0) {
            acc = 0.f;
#pragma unroll
            for (int g = 0; g < 16; ++g)
                if (g < G) acc += __expf(x[e][g] - hm[g]);
        } else {
            acc = x[e][0];
#pragma unroll
            for (int g = 1; g < 16; ++g)
                if (g < G) acc = fmaxf(acc, x[e][g]);
        }
        score[rk * (long)MP + p] = acc;
        keys[p - c0] = f2u(acc);
    }
    lds_barrier();

    const int lo_c = min(max(n_sink, c0), c1) - c0;       // selectable slice of
    const int hi_c = max(min(n_sel_hi, c1), c0) - c0;     // this chunk, local idx
    const int n_loc = max(hi_c - lo_c, 0);

    if (final_mode) {
        // the whole row lives in this chunk: finish here
        if (keep_all || b >= n_sel) {
            fill_all_pages(trow, max(n_pages, 0), MP, true);
            if (tid == 0) page_cnt[rk] = max(n_pages, 0);
            return;
        }
        const uint32_t tau = block_kth_largest<SEL_BLK>(keys + lo_c, n_loc, b, hist, s3);
        const int nsel_w = emit_topk<SEL_BLK>(keys + lo_c, n_loc, b, tau,
                                              [&](int i) { return n_sink + i; },
                                              trow + n_sink, nullptr, wsum);
        const int cnt = n_sink + nsel_w + (n_pages - n_sel_hi);
        for (int i = tid; i < MP; i += SEL_BLK) {
            if (i < n_sink) trow[i] = i;
            else if (i >= n_sink + nsel_w && i < cnt) trow[i] = n_sel_hi + (i - n_sink - nsel_w);
            else if (i >= cnt) trow[i] = -1;
        }
        if (tid == 0) page_cnt[rk] = cnt;
        return;
    }

    // ---- multi-chunk: emit this chunk's local top-min(b, n_loc) ----------
    uint32_t* ck = cand_key + (rk * Z1 + z) * (long)SEL_CH;
    int* cp = cand_page + (rk * Z1 + z) * (long)SEL_CH;
    int ncand = 0;
    if (!keep_all && n_loc > 0) {
        const int k_loc = min(b, n_loc);
        uint32_t tau = 0u;   // k_loc == n_loc: every key >= 0 is kept
        if (k_loc < n_loc) tau = block_kth_largest<SEL_BLK>(keys + lo_c, n_loc, k_loc, hist, s3);
        const int base = c0 + lo_c;
        ncand = emit_topk<SEL_BLK>(keys + lo_c, n_loc, k_loc, tau,
                                   [&](int i) { return base + i; }, cp, ck, wsum);
    }
    if (tid == 0) cand_cnt[rk * Z1 + z] = ncand;
}

// ---------------------------------------------------------------------------
// finishing kernel (multi-chunk rows)
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// finishing kernel (rows spanning several chunks)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(FIN_BLK) void sel_finish_kernel(
    const int* __restrict__ npg, const int* __restrict__ nsh, const int* __restrict__ bfix,
    int* __restrict__ page_table, int* __restrict__ page_cnt,
    const uint32_t* __restrict__ cand_key, const int* __restrict__ cand_page,
    const int* __restrict__ cand_cnt, uint32_t* __restrict__ spill_key, int* __restrict__ spill_page,
    int n_sink, int MP, int Z1)
{
    const int kh = blockIdx.y, r = blockIdx.z;
    const long rk = (long)r * gridDim.y + kh;
    const int n_pages = min(npg[r], MP);
    const int n_sel_hi = min(nsh[r], MP);
    const int n_sel = n_sel_hi - n_sink;
    int b = bfix[r];
    b = max(1, min(b, max(n_sel, 1)));
    int* trow = page_table + rk * (long)MP;
    if (n_sel <= 1 || b >= n_sel) {
        for (int i = threadIdx.x; i < max(n_pages, 0); i += FIN_BLK) trow[i] = i;
        if (threadIdx.x == 0) page_cnt[rk] = max(n_pages, 0);
        return;
    }
    __shared__ int offs[FIN_MAXZ + 1];
    __shared__ uint32_t lkey[FIN_CAP];
    __shared__ int lpage[FIN_CAP];
    __shared__ int hist[256];
    __shared__ int s3[4];
    __shared__ int wsum[FIN_BLK / kWave + 1];
    finish_row<FIN_BLK>(rk, n_pages, n_sel_hi, n_sink, b, MP, Z1, trow, page_cnt + rk, cand_key,
                        cand_page, cand_cnt, spill_key, spill_page, offs, lkey, lpage, hist, s3,
                        wsum);
}

// ---------------------------------------------------------------------------
// page-parallel route with register-resident keys (rows > ROW_MAXP pages):
// sel_chunk2_kernel: one 1024-thread workgroup per 2048-page chunk, 2 pages
// per thread (measured faster than 512 x 4: less serial work per thread); sel_finish2_kernel: one 1024-thread workgroup per row holds up
// to 4096 candidates (4 per thread) in registers.
// ---------------------------------------------------------------------------
constexpr int C2_BLK = 1024;
constexpr int C2_E = SEL_CH / C2_BLK;                  // 2
static_assert(C2_E == 2, "sel_chunk2_kernel loads and stores its pages as float2");
constexpr int F2_BLK = 1024;
constexpr int F2_CAP = F2_BLK * 16;                    // register-resident candidates

// BAND = false: emit the chunk's local top-min(b, n) candidates.
// BAND = true (large budgets): add the chunk's key histogram (top 12 bits)
// into the row's global histogram instead; sel_band_kernel then emits the
// candidates at or above the row's boundary bin.
// GL: heads loaded per thread (>= G; the host picks 1, 4, 8 or 16), so
// small groups issue no clamped duplicate loads.
template <bool BAND, int E = C2_E, int GL = 16>
__global__ __launch_bounds__(C2_BLK) void sel_chunk2_kernel(
    const float* __restrict__ score_h, const float* __restrict__ pmax, int Zs,
    const int* __restrict__ npg, const int* __restrict__ nsh, const int* __restrict__ bfix,
    float* __restrict__ score, int* __restrict__ page_table,
    uint32_t* __restrict__ cand_key, int* __restrict__ cand_page, int* __restrict__ cand_cnt,
    int* __restrict__ ghist, int n_sink, int MP, int G, int combine)
{
    const int z = blockIdx.x, kh = blockIdx.y, r = blockIdx.z;
    const int n_kv = gridDim.y, Z1 = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long rk = (long)r * n_kv + kh;
    const int n_sel_hi = min(nsh[r], MP);
    static_assert(E == 1 || E == 2, "one or two pages per thread");
    static_assert(!BAND || E == C2_E, "the band route keeps 2048-page chunks");
    constexpr int CH = E * C2_BLK;                      // pages per chunk
    const int c0 = z * CH;
    const int p0 = c0 + E * tid;                        // this thread's E pages

    __shared__ float hm[16];
    __shared__ int hist[4096];
    __shared__ int wtot[C2_BLK / kWave];
    __shared__ int s3[4];
    __shared__ int wsum[C2_BLK / kWave + 1];

    // score_h of every head in flight first (row-bounded, no parameter wait)
    const float* shb = score_h + rk * (long)G * MP;
    float2 xv[GL];
#pragma unroll
    for (int g = 0; g < GL; ++g) {                       // clamped, unconditional (see the row kernel)
        if constexpr (E == 2)
            xv[g] = *reinterpret_cast<const float2*>(shb + (long)min(g, G - 1) * MP + min(p0, MP - 2));
        else
            xv[g] = make_float2(shb[(long)min(g, G - 1) * MP + min(p0, MP - 1)], 0.f);
    }
    int* trow = page_table + rk * (long)MP;
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (p0 + e < MP) trow[p0 + e] = -1;
    if (combine == 0) {
        // the radix histogram is zeroed ahead of this barrier (the local
        // selection then needs no barrier of its own before its first pass)
        if constexpr (!BAND) {
            for (int i = tid; i < 4096; i += C2_BLK) hist[i] = 0;
            if (tid == 0) s3[3] = 0;
        }
        for (int g = wave; g < G; g += C2_BLK / kWave) {
            const float m = wave_max(chunk_max(pmax + (rk * 16 + g) * Zs, Zs));
            if (lane == 0) hm[g] = m;
        }
        lds_barrier();
    }
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) acc[e] = (combine == 0) ? 0.f : -INFINITY;
    // combine mode tested once, heads past G masked by selects (see the row
    // kernel)
    if (combine == 0) {
#pragma unroll
        for (int g = 0; g < GL; ++g) {
            const float x4[2] = {xv[g].x, xv[g].y};
            const float h = hm[min(g, G - 1)];
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float t = __expf(x4[e] - h);
                acc[e] = (g < G) ? acc[e] + t : acc[e];
            }
        }
    } else {
#pragma unroll
        for (int g = 0; g < GL; ++g) {
            const float x4[2] = {xv[g].x, xv[g].y};
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float mx = (g == 0) ? x4[e] : fmaxf(acc[e], x4[e]);
                acc[e] = (g < G) ? mx : acc[e];
            }
        }
    }
    const int pend = max(n_sel_hi, 0);
    float* srow = score + rk * (long)MP;
    if constexpr (E == 2) {
        if (p0 + E <= pend) {
            *reinterpret_cast<float2*>(srow + p0) = make_float2(acc[0], acc[E - 1]);
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e)
                if (p0 + e < pend) srow[p0 + e] = acc[e];
        }
    } else {
        if (p0 < pend) srow[p0] = acc[0];
    }
    const int n_sel = n_sel_hi - n_sink;
    int b = bfix[r];
    b = max(1, min(b, max(n_sel, 1)));
    uint32_t key[E];
    bool val[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int p = p0 + e;
        val[e] = (n_sel > 1) && p >= n_sink && p < n_sel_hi;
        key[e] = f2u(acc[e]);
    }
    if constexpr (BAND) {
        for (int i = tid; i < 4096; i += C2_BLK) hist[i] = 0;
        lds_barrier();
#pragma unroll
        for (int e = 0; e < E; ++e) hist_add(hist, (int)(key[e] >> 20), val[e]);
        lds_barrier();
        int* gh = ghist + rk * 4096;
        for (int i = tid; i < 4096; i += C2_BLK)
            if (hist[i]) __hip_atomic_fetch_add(gh + i, hist[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // valid pages of the chunk: [max(c0, n_sink), min(c0 + CH, n_sel_hi))
    const int n_loc = (n_sel > 1) ? max(0, min(c0 + CH, n_sel_hi) - max(c0, n_sink)) : 0;
    uint32_t* ck = cand_key + (rk * Z1 + z) * (long)SEL_CH;
    int* cp = cand_page + (rk * Z1 + z) * (long)SEL_CH;
    int ncand = 0;
    if (n_loc > 0) {
        const int k_loc = min(b, n_loc);
        RadixSel rs{0u, 0u, 0, true};                    // k_loc == n_loc: keep every valid key (>= 0)
        // nrm keys are sums of G terms <= 1: 2G bounds them (see the row
        // kernel); the histogram was zeroed before the head-max barrier
        if (k_loc < n_loc)
            rs = reg_kth_largest<C2_BLK, E>(key, val, k_loc, hist, wtot, s3,
                                            combine == 0 ? f2u(2.f * (float)G) : 0u);
        ncand = reg_emit<C2_BLK, E, false>(key, val, rs, wsum, [&](int pos, int e) {
            ck[pos] = key[e];
            cp[pos] = p0 + e;
        });
    }
    if (tid == 0) cand_cnt[rk * Z1 + z] = ncand;
}

// Exact b-th largest over register-resident candidates (thread order = page
// order), ordered emission, sink / window, page count.
template <int E>
__device__ void finish2_select(long rk, int b, int n_sink, int n_pages, int n_sel_hi,
                               int* __restrict__ trow, int* __restrict__ page_cnt,
                               const uint32_t (&key)[E], const int (&page)[E], const bool (&val)[E],
                               int* hist, int* wtot, int* s3, int* wsum) {
    const int tid = threadIdx.x;
    // (the candidate lists of the chunks: the boundary-bin compaction
    // measured slower here than the histogram passes, 9.2 vs 6.4 us at 1M)
    const RadixSel rs = reg_kth_largest<F2_BLK, E, false>(key, val, b, hist, wtot, s3);
    reg_emit<F2_BLK, E>(key, val, rs, wsum, [&](int pos, int e) { trow[n_sink + pos] = page[e]; });
    const int cnt = n_sink + b + (n_pages - n_sel_hi);
    for (int i = tid; i < n_sink; i += F2_BLK) trow[i] = i;
    for (int i = n_sink + b + tid; i < cnt; i += F2_BLK) trow[i] = n_sel_hi + (i - n_sink - b);
    if (tid == 0) page_cnt[rk] = cnt;
}

// Candidates j = E t .. E t + E - 1 of the chunk-ordered (= page-ordered)
// list, located by a binary search over the chunk offsets.
template <int E>
__device__ void finish2_regs(long rk, int N, int Z1, int b, int n_sink, int n_pages,
                             int n_sel_hi, int* __restrict__ trow, int* __restrict__ page_cnt,
                             const uint32_t* __restrict__ cand_key, const int* __restrict__ cand_page,
                             const int* offs, int* hist, int* wtot, int* s3, int* wsum) {
    const int tid = threadIdx.x;
    uint32_t key[E];
    int page[E];
    bool val[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int j = E * tid + e;
        val[e] = j < N;
        key[e] = 0u;
        page[e] = 0;
        if (val[e]) {
            int lo = 0, hi = Z1;                            // offs[lo] <= j < offs[hi]
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (offs[mid] <= j) lo = mid; else hi = mid;
            }
            const long src = (rk * Z1 + lo) * (long)SEL_CH + (j - offs[lo]);
            key[e] = cand_key[src];
            page[e] = cand_page[src];
        }
    }
    finish2_select<E>(rk, b, n_sink, n_pages, n_sel_hi, trow, page_cnt, key, page, val, hist, wtot,
                      s3, wsum);
}


// Large-budget route, second pass: every chunk reads its row's key histogram
// (complete after sel_chunk2_kernel<true>), finds the boundary bin T (the bin
// holding the b-th largest key) and emits, in page order, its pages whose
// key's top 12 bits are >= T -- every globally kept page plus the rest of
// bin T -- for sel_finish2_kernel.  Keys are re-read from `score`.
__global__ __launch_bounds__(C2_BLK) void sel_band_kernel(
    const int* __restrict__ nsh, const int* __restrict__ bfix, const float* __restrict__ score,
    uint32_t* __restrict__ cand_key, int* __restrict__ cand_page, int* __restrict__ cand_cnt,
    const int* __restrict__ ghist, int n_sink, int MP)
{
    const int z = blockIdx.x, kh = blockIdx.y, r = blockIdx.z;
    const int n_kv = gridDim.y, Z1 = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const long rk = (long)r * n_kv + kh;
    const int n_sel_hi = min(nsh[r], MP);
    const int n_sel = n_sel_hi - n_sink;
    int b = bfix[r];
    b = max(1, min(b, max(n_sel, 1)));
    __shared__ int wtot[C2_BLK / kWave];
    __shared__ int wsum[C2_BLK / kWave + 1];
    __shared__ int tbin;
    if (n_sel <= 1 || b >= n_sel) {                     // keep-all rows need no candidates
        if (tid == 0) cand_cnt[rk * Z1 + z] = 0;
        return;
    }
    // boundary bin: thread t holds bins top .. top - BPT + 1 (top = 4095 - BPT t),
    // ascending threads = descending bins
    constexpr int BPT = 4096 / C2_BLK;
    const int top = 4095 - BPT * tid;
    int c = 0, hb[BPT];
    const int* gh = ghist + rk * 4096;
#pragma unroll
    for (int j = 0; j < BPT; ++j) { hb[j] = gh[top - j]; c += hb[j]; }
    const int incl = wave_incl_scan_i(c);
    if (lane == kWave - 1) wtot[wave] = incl;
    lds_barrier();
    const int base = wave_sum_i((lane < wave) ? wtot[lane] : 0);
    const int above0 = base + incl - c;
    if (c > 0 && above0 < b && b <= base + incl) {
        int above = above0;
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
            if (above + hb[j] >= b) { tbin = top - j; break; }
            above += hb[j];
        }
    }
    lds_barrier();
    const uint32_t T = (uint32_t)tbin;
    const int p0 = z * SEL_CH + C2_E * tid;
    uint32_t key[C2_E];
    int nv = 0;
    bool kp[C2_E];
    const float* srow = score + rk * (long)MP;
#pragma unroll
    for (int e = 0; e < C2_E; ++e) {
        const int p = p0 + e;
        const bool v = p >= n_sink && p < n_sel_hi;
        key[e] = v ? f2u(srow[p]) : 0u;
        kp[e] = v && (key[e] >> 20) >= T;
        nv += kp[e];
    }
    int tot;
    int pos = block_excl_scan<C2_BLK>(nv, wsum, tot);
    const long cb = (rk * Z1 + z) * (long)SEL_CH;
#pragma unroll
    for (int e = 0; e < C2_E; ++e)
        if (kp[e]) { cand_key[cb + pos] = key[e]; cand_page[cb + pos] = p0 + e; ++pos; }
    if (tid == 0) cand_cnt[rk * Z1 + z] = tot;
}

__global__ __launch_bounds__(F2_BLK) void sel_finish2_kernel(
    const int* __restrict__ npg, const int* __restrict__ nsh, const int* __restrict__ bfix,
    int* __restrict__ page_table, int* __restrict__ page_cnt,
    const uint32_t* __restrict__ cand_key, const int* __restrict__ cand_page,
    const int* __restrict__ cand_cnt, uint32_t* __restrict__ spill_key, int* __restrict__ spill_page,
    int* __restrict__ ghist, int n_sink, int MP, int Z1)
{
    const int kh = blockIdx.y, r = blockIdx.z;
    const long rk = (long)r * gridDim.y + kh;
    const int tid = threadIdx.x;
    if (ghist)                          // large-budget route: leave the row histogram zeroed
        for (int i = tid; i < 4096; i += F2_BLK) ghist[rk * 4096 + i] = 0;
    const int n_pages = min(npg[r], MP);
    const int n_sel_hi = min(nsh[r], MP);
    const int n_sel = n_sel_hi - n_sink;
    int b = bfix[r];
    b = max(1, min(b, max(n_sel, 1)));
    int* trow = page_table + rk * (long)MP;
    if (n_sel <= 1 || b >= n_sel) {
        for (int i = tid; i < max(n_pages, 0); i += F2_BLK) trow[i] = i;
        if (tid == 0) page_cnt[rk] = max(n_pages, 0);
        return;
    }
    __shared__ int offs[FIN_MAXZ + 1];
    __shared__ int hist[4096];
    __shared__ int wtot[F2_BLK / kWave];
    __shared__ int s3[4];
    __shared__ int wsum[F2_BLK / kWave + 1];
    // Slotted layout (the usual small budget): chunk z's local top-b list (at
    // most min(b, SEL_CH) candidates, page-ordered) maps onto ceil(that / 4)
    // consecutive threads, 4 slots each, so thread order is page order and the
    // counts load in the same round trip as the candidates (no offset scan).
    // Only on the local-top-b route (no histogram): band lists can be longer.
    // (4 slots per thread; 8 when the lists need more than the workgroup's
    // threads at 4, e.g. 64 chunks of 1024 pages at 1M)
    auto slotted = [&](auto slots) {
        constexpr int SL = decltype(slots)::value;
        const int tpc = cdiv(min(b, SEL_CH), SL);          // threads per chunk list
        const int z = tid / tpc, sl = (tid - z * tpc) * SL;
        const bool zin = z < Z1;
        const long src = (rk * Z1 + (zin ? z : 0)) * (long)SEL_CH + sl;
        const int czl = cand_cnt[rk * Z1 + (zin ? z : 0)];
        uint32_t key[SL];
        int page[SL];
        bool val[SL];
#pragma unroll
        for (int e = 0; e < SL; ++e) {                     // slots past the count are masked
            key[e] = cand_key[src + e];
            page[e] = cand_page[src + e];
        }
        const int cz = zin ? czl : 0;
#pragma unroll
        for (int e = 0; e < SL; ++e) {
            val[e] = zin && sl + e < cz;
            if (!val[e]) key[e] = 0u;
        }
        finish2_select<SL>(rk, b, n_sink, n_pages, n_sel_hi, trow, page_cnt, key, page, val, hist,
                           wtot, s3, wsum);
    };
    if (!ghist && (long)Z1 * cdiv(min(b, SEL_CH), 4) <= F2_BLK) {
        slotted(std::integral_constant<int, 4>{});
        return;
    }
    if (!ghist && (long)Z1 * cdiv(min(b, SEL_CH), 8) <= F2_BLK) {
        slotted(std::integral_constant<int, 8>{});
        return;
    }
    {
        const int c = (tid < Z1) ? cand_cnt[rk * Z1 + tid] : 0;
        int tot;
        const int ex = block_excl_scan<F2_BLK>(c, wsum, tot);
        if (tid < Z1) offs[tid] = ex;
        if (tid == 0) offs[Z1] = tot;
        lds_barrier();
    }
    const int N = offs[Z1];
    if (N > F2_CAP) {                   // more candidates than registers: global spill
        finish_row<F2_BLK>(rk, n_pages, n_sel_hi, n_sink, b, MP, Z1, trow, page_cnt + rk, cand_key,
                           cand_page, cand_cnt, spill_key, spill_page, offs, nullptr, nullptr, hist,
                           s3, wsum, 0);
        return;
    }
    if (N <= F2_BLK * 4)
        finish2_regs<4>(rk, N, Z1, b, n_sink, n_pages, n_sel_hi, trow, page_cnt, cand_key,
                        cand_page, offs, hist, wtot, s3, wsum);
    else
        finish2_regs<16>(rk, N, Z1, b, n_sink, n_pages, n_sel_hi, trow, page_cnt, cand_key,
                         cand_page, offs, hist, wtot, s3, wsum);
}

// ---------------------------------------------------------------------------
// derive (select.py:28-58)
// ---------------------------------------------------------------------------
__global__ void derive_kernel(const int* __restrict__ seq_lens, int n_req, int page, int window,
                              int sink, int budget_abs, double budget, int* __restrict__ npg_o,
                              int* __restrict__ nsh_o, int* __restrict__ b_o) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_req; i += gridDim.x * blockDim.x) {
        const int sl = seq_lens[i];
        const int npg = (sl + page - 1) / page;
        const int nsh = npg - window;
        const int s = nsh - sink;
        int b;
        if (budget_abs > 0) {
            b = min(budget_abs, max(s, 1));
            b = max(b, 1);
        } else {
            const double bf = ceil((double)s * budget);
            b = min(max((int)bf, 1), max(s, 1));
        }
        npg_o[i] = npg;
        nsh_o[i] = nsh;
        b_o[i] = b;
    }
}

}  // namespace locks

using namespace locks;

// Workspace bytes of one (request, kv head) row: candidate keys + pages per
// chunk slot, spill keys + pages per page, per-chunk counts, and the
// large-budget route's 4096-bin row histogram.
static long sel_row_bytes(long Z1, long max_pages) {
    return Z1 * SEL_CH * 8 + max_pages * 8 + Z1 * 4 + 4096 * 4;
}

// Chunk lists are laid out for the largest chunk count any route uses: the
// 1024-page chunks of the small-budget page-parallel route (each list keeps
// its SEL_CH-entry slot).
constexpr int SEL_CH_MIN = SEL_CH / 2;

extern "C" int64_t locks_select_workspace_bytes(int32_t n_req, int32_t n_kv, int32_t max_pages) {
    if (n_req < 0 || n_kv < 1 || max_pages < 1) return -1;
    const long Z1 = cdiv(max_pages, SEL_CH_MIN);
    const long rows = (long)n_req * n_kv;
    const long bytes = rows * sel_row_bytes(Z1, max_pages);
    return (bytes + 255) / 256 * 256;
}

extern "C" int32_t locks_select_nrm_topb(
    const float* score_h, const float* page_max, int32_t score_chunks,
    const int32_t* n_pages, const int32_t* n_sel_hi, const int32_t* b_fix,
    float* score, int32_t* page_table, int32_t* page_cnt,
    void* workspace, int64_t workspace_bytes,
    int32_t n_req, int32_t n_kv, int32_t G, int32_t n_sink, int32_t max_pages,
    int32_t combine, int32_t b_max, void* stream)
{
    LOCKS_REQUIRE(G >= 1 && G <= 16, "locks_select_nrm_topb: G=%d outside [1, 16]", G);
    LOCKS_REQUIRE(n_req >= 0 && n_kv >= 1 && max_pages >= 1, "locks_select_nrm_topb: bad geometry");
    LOCKS_REQUIRE(n_sink >= 0, "locks_select_nrm_topb: n_sink=%d < 0", n_sink);
    LOCKS_REQUIRE(combine == 0 || combine == 1, "locks_select_nrm_topb: combine must be 0 (nrm) or 1 (max)");
    LOCKS_REQUIRE(combine == 1 || (page_max && score_chunks >= 1),
                  "locks_select_nrm_topb: nrm combine needs the scorer's page maxima");
    LOCKS_REQUIRE(score_h && n_pages && n_sel_hi && b_fix && score && page_table && page_cnt,
                  "locks_select_nrm_topb: null pointer argument");
    const int Z1 = cdiv(max_pages, SEL_CH);
    LOCKS_REQUIRE(Z1 <= FIN_MAXZ, "locks_select_nrm_topb: max_pages=%d exceeds %d", max_pages, FIN_MAXZ * SEL_CH);
    const int64_t need = locks_select_workspace_bytes(n_req, n_kv, max_pages);
    LOCKS_REQUIRE(Z1 == 1 || (workspace && workspace_bytes >= need),
                  "locks_select_nrm_topb: workspace %lld B < required %lld B",
                  (long long)workspace_bytes, (long long)need);
    if (n_req == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    // Every region is laid out for the workspace's row capacity, not for this
    // call's n_req: the band route's row histograms must stay zero between
    // calls (the finisher clears them), so they may never move onto bytes a
    // call with another batch size used for candidates.
    const long ZW = cdiv(max_pages, SEL_CH_MIN);           // chunk slots per row in the layout
    const long cap = workspace ? (long)(workspace_bytes / sel_row_bytes(ZW, max_pages)) : 0;
    uint8_t* ws = (uint8_t*)workspace;
    uint32_t* cand_key = (uint32_t*)ws;
    int* cand_page = (int*)(ws + cap * ZW * SEL_CH * 4);
    uint32_t* spill_key = (uint32_t*)(ws + cap * ZW * SEL_CH * 8);
    int* spill_page = (int*)(ws + cap * ZW * SEL_CH * 8 + cap * (long)max_pages * 4);
    int* cand_cnt = (int*)(ws + cap * ZW * SEL_CH * 8 + cap * (long)max_pages * 8);
    int* ghist = cand_cnt + cap * ZW;
    // A whole row's score_h (G x pages x 4 B) goes through one CU in the row
    // kernel; above 64K (head, page) entries the page-parallel chunk route
    // wins (GLM G = 16, measured per step: 8192 pages 1.485 -> 1.400 ms;
    // 4096 pages 1.202 row vs 1.355 chunk)
#ifndef SEL_ROW_MAX_GP
#define SEL_ROW_MAX_GP 65536L
#endif
    // The row kernel also serves rows of one chunk or less: against the
    // single-chunk kernel it measured GLM 16K 1.225 -> 1.083 ms and 32K
    // 1.327 -> 1.104 ms per step
    if (max_pages <= ROW_MAXP && max_pages % 4 == 0 &&
        (long)G * max_pages <= SEL_ROW_MAX_GP) {
#define ROW_LAUNCH(EV, HBV)                                                                \
        hipLaunchKernelGGL((sel_row_kernel<EV, HBV>), dim3(n_kv, n_req), dim3(ROW_BLK), 0, st, score_h, \
                           page_max, score_chunks, n_pages, n_sel_hi, b_fix, score, page_table, \
                           page_cnt, n_sink, max_pages, G, combine)
        // heads per load batch: no clamped duplicate loads for one head (MLA)
        // or groups of at most 4 (Llama G = 4: 16 -> 8 loads per thread)
        if (max_pages <= 4 * ROW_BLK) {
            if (G == 1) ROW_LAUNCH(4, 1);
            else if (G <= 4) ROW_LAUNCH(4, 4);
            else ROW_LAUNCH(4, 8);
        } else {
            if (G == 1) ROW_LAUNCH(8, 1);
            else if (G <= 4) ROW_LAUNCH(8, 4);
            else ROW_LAUNCH(8, 8);
        }
#undef ROW_LAUNCH
        return check_launch("sel_row_kernel");
    }
    if (Z1 > 1 && max_pages % 4 == 0) {
        // Local top-b lists of every chunk past the 4-per-thread finisher:
        // the histogram (band) route is faster (measured at 256K..1M with
        // b = 1638..6553: 25-36 us against 40-160 us).
        const bool band = (long)b_max * Z1 > F2_BLK * 4;
        // With a small budget and a wide GQA group, 1024-page chunks (one page
        // per thread) halve the score_h each workgroup pulls through its CU
        // (G x 4 KB), while the finisher's lists still fit its slotted
        // layout, at 8 slots per thread when 4 do not fit (GLM G = 16, measured
        // per step: 128K 1.379 -> 1.285 ms, 256K 1.530 -> 1.440, 512K 1.791 ->
        // 1.708, ragged batch 2.047 -> 1.977; 1M, 64 chunks: 2.297 -> 2.25-2.27)
        const int Zs = cdiv(max_pages, SEL_CH_MIN);
        const bool small_chunks = !band && G > 4 && (long)Zs * cdiv(min(b_max, SEL_CH), 8) <= F2_BLK;
        // heads loaded per thread: the group rounded up to 1, 4, 8 or 16
        const int gl = G == 1 ? 1 : G <= 4 ? 4 : G <= 8 ? 8 : 16;
#define C2_LAUNCH(BANDV, EV, ZV, HISTV)                                                              \
        do {                                                                                          \
            auto go = [&](auto glc) {                                                                 \
                hipLaunchKernelGGL((sel_chunk2_kernel<BANDV, EV, decltype(glc)::value>), dim3(ZV, n_kv, n_req), \
                                   dim3(C2_BLK), 0, st, score_h, page_max, score_chunks, n_pages,     \
                                   n_sel_hi, b_fix, score, page_table, cand_key, cand_page, cand_cnt, \
                                   HISTV, n_sink, max_pages, G, combine);                            \
            };                                                                                        \
            if (gl == 1) go(std::integral_constant<int, 1>{});                                        \
            else if (gl == 4) go(std::integral_constant<int, 4>{});                                   \
            else if (gl == 8) go(std::integral_constant<int, 8>{});                                   \
            else go(std::integral_constant<int, 16>{});                                               \
        } while (0)
        if (small_chunks) {
            C2_LAUNCH(false, 1, Zs, nullptr);
            int rc = check_launch("sel_chunk2_kernel<small>");
            if (rc) return rc;
            hipLaunchKernelGGL(sel_finish2_kernel, dim3(1, n_kv, n_req), dim3(F2_BLK), 0, st,
                               n_pages, n_sel_hi, b_fix, page_table, page_cnt, cand_key, cand_page,
                               cand_cnt, spill_key, spill_page, nullptr, n_sink, max_pages, Zs);
            return check_launch("sel_finish2_kernel");
        }
        if (band) {
            C2_LAUNCH(true, C2_E, Z1, ghist);
            int rc = check_launch("sel_chunk2_kernel<band>");
            if (rc) return rc;
            hipLaunchKernelGGL(sel_band_kernel, dim3(Z1, n_kv, n_req), dim3(C2_BLK), 0, st,
                               n_sel_hi, b_fix, score, cand_key, cand_page, cand_cnt, ghist, n_sink,
                               max_pages);
            rc = check_launch("sel_band_kernel");
            if (rc) return rc;
        } else {
            C2_LAUNCH(false, C2_E, Z1, nullptr);
            int rc = check_launch("sel_chunk2_kernel");
            if (rc) return rc;
        }
        hipLaunchKernelGGL(sel_finish2_kernel, dim3(1, n_kv, n_req), dim3(F2_BLK), 0, st,
                           n_pages, n_sel_hi, b_fix, page_table, page_cnt, cand_key, cand_page,
                           cand_cnt, spill_key, spill_page, band ? ghist : nullptr, n_sink,
                           max_pages, Z1);
        return check_launch("sel_finish2_kernel");
#undef C2_LAUNCH
    }
    hipLaunchKernelGGL(sel_chunk_kernel, dim3(Z1, n_kv, n_req), dim3(SEL_BLK), 0, st,
                       score_h, page_max, score_chunks, n_pages, n_sel_hi, b_fix, score,
                       page_table, page_cnt, cand_key, cand_page, cand_cnt, n_sink,
                       max_pages, G, combine);
    int rc = check_launch("sel_chunk_kernel");
    if (rc || Z1 == 1) return rc;
    hipLaunchKernelGGL(sel_finish_kernel, dim3(1, n_kv, n_req), dim3(FIN_BLK), 0, st,
                       n_pages, n_sel_hi, b_fix, page_table, page_cnt, cand_key, cand_page,
                       cand_cnt, spill_key, spill_page, n_sink, max_pages, Z1);
    return check_launch("sel_finish_kernel");
}

extern "C" int32_t locks_derive_params(const int32_t* seq_lens, int32_t n_req, int32_t page,
                                       int32_t window_pages, int32_t sink_pages,
                                       int32_t budget_abs, double budget, int32_t* n_pages,
                                       int32_t* n_sel_hi, int32_t* b_fix, void* stream) {
    LOCKS_REQUIRE(page >= 1 && window_pages >= 1 && sink_pages >= 0,
                  "locks_derive_params: bad page=%d window=%d sink=%d", page, window_pages, sink_pages);
    LOCKS_REQUIRE(budget_abs > 0 || (budget > 0.0 && budget <= 1.0),
                  "locks_derive_params: budget %f outside (0, 1] with no absolute budget", budget);
    LOCKS_REQUIRE(seq_lens && n_pages && n_sel_hi && b_fix, "locks_derive_params: null pointer argument");
    if (n_req <= 0) return 0;
    const int blk = 256, grid = cdiv(n_req, blk);
    hipLaunchKernelGGL(derive_kernel, dim3(grid), dim3(blk), 0, (hipStream_t)stream, seq_lens,
                       n_req, page, window_pages, sink_pages, budget_abs, budget, n_pages,
                       n_sel_hi, b_fix);
    return check_launch("derive_kernel");
}
