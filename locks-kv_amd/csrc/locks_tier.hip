// DRAM tier control plane on gfx950: per-step staging lifecycle and per-layer
// exact-LRU hot-buffer residency (reference src/locks/tier/staging.py and
// tier/residency.py).  The decode reads each selected page from the hot
// buffer, the staging pool or the pinned host pool (locks_decode.hip, TIER);
// these kernels decide which pages sit where and move the bytes.
//
//   locks_tier_invalidate   residency.py:271-307   pages written this step lose
//                                                  hot residency and pool validity
//   locks_tier_stage_begin  staging.py:125-244     flushed-latch clear, collect +
//                                                  free of complete staged pages,
//                                                  staging-block allocation, slot map
//   locks_tier_flush_copy   staging.py:247-277     collected pages -> pinned pool
//   locks_tier_scatter      staging.py:57-82       this step's V (K) -> staging pool
//   locks_tier_plan         residency.py:51-145    hit/miss of the selected pages,
//                                                  exact-LRU victims, map install
//   locks_tier_fetch        residency.py:216-268   miss pages -> their hot slots
//
// Serial reference loops become one workgroup with block scans: every order
// the reference fixes (requests in order, pages in order inside a request,
// victims by (lru clock, slot)) is kept exactly; orders it leaves to atomics
// (flush list, free-stack pushes, fetch list) are fixed to page / install order.
// State mutated inside a kernel and re-read by other waves is only ever
// shared within one workgroup, whose waves run on one CU and share its
// write-through L1: workgroup barriers order it.  Values produced by
// atomics (executed at the L2) are re-read with agent-scope loads.  (An
// agent-scope release would write back the L2 at every phase: measured
// +15 us per layer.)
#include <climits>

#include "locks_common.h"
#include "locks_hip.h"

namespace locks {
namespace {

constexpr int TB = 1024;                 // threads of the one-workgroup kernels
constexpr int TB_WAVES = TB / kWave;
constexpr int TP_KMAX = 4096;            // victims ranked per round in LDS
constexpr int TP_BINS = 2048;            // radix histogram of the LRU clocks

__device__ __forceinline__ void phase_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

__device__ __forceinline__ int ld_coh(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exclusive prefix of v over the workgroup (thread order); *total = sum.
__device__ __forceinline__ int block_scan_excl(int v, int* wsum, int* total) {
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x >> 6;
    const int inc = wave_incl_scan_i(v);
    if (lane == kWave - 1) wsum[w] = inc;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < TB_WAVES; ++i) {
        const int s = wsum[i];
        off += (i < w) ? s : 0;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return off + inc - v;
}

// 16-byte copy of one page (elems bf16, contiguous) by one wave.
__device__ __forceinline__ void wave_copy(uint16_t* dst, const uint16_t* src, long elems, int lane) {
    for (long c = lane; c * 8 < elems; c += kWave)
        *reinterpret_cast<uint4*>(dst + c * 8) = *reinterpret_cast<const uint4*>(src + c * 8);
}

// ---------------------------------------------------------------------------
// invalidate (residency.py:271-307): grid (n_req), every (page, layer, kv).
// The guard is seq_len > 0 only, as in the reference.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tier_invalidate_kernel(
    const int* __restrict__ bt, long bt_sr, int bt_cols, const int* __restrict__ sl,
    const int* __restrict__ qsl, int* p2s, int* s2p, int8_t* pool_valid, int L, int n_kv, int NB,
    int S, int page)
{
    const int r = blockIdx.x;
    const int s = sl[r];
    if (s <= 0) return;
    const int ql = qsl[r + 1] - qsl[r];
    const int p0 = max((s - ql) / page, 0), p1 = min((s - 1) / page, bt_cols - 1);
    const int rows = L * n_kv;
    const long n = (long)max(p1 - p0 + 1, 0) * rows;
    for (long e = threadIdx.x; e < n; e += blockDim.x) {
        const int p = p0 + (int)(e / rows), row = (int)(e % rows);
        const int blk = bt[(long)r * bt_sr + p];
        if (blk < 0 || blk >= NB) continue;
        const long ix = (long)row * NB + blk;
        pool_valid[ix] = 0;
        const int slot = p2s[ix];
        if (slot >= 0 && slot < S) s2p[(long)row * S + slot] = -1;
        if (slot != -1) p2s[ix] = -1;
    }
}

// ---------------------------------------------------------------------------
// staging lifecycle (staging.py:373-442 order): one workgroup.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(TB) void tier_stage_begin_kernel(
    const int* __restrict__ bt, long bt_sr, int bt_cols, const int* __restrict__ sl,
    const int* __restrict__ qsl, int n_req, int* vbo, int* vfl, int* stack, int* top_p,
    int* flist, int* fcnt_p, int max_flush, long long* vslot, int max_tokens, int* overflow,
    int NB, int NV, int page)
{
    __shared__ int wsum[TB_WAVES];
    const int tid = threadIdx.x;
    for (int t = tid; t < max_tokens; t += TB) vslot[t] = -1;
    // vflush_clear (:125-138): pages written this step lose the flushed latch
    for (int r = 0; r < n_req; ++r) {
        const int s = sl[r], ql = qsl[r + 1] - qsl[r];
        if (s <= 0 || ql <= 0) continue;
        const int p0 = (s - ql) / page, p1 = min((s - 1) / page, bt_cols - 1);
        for (int p = p0 + tid; p <= p1; p += TB) {
            const int blk = bt[(long)r * bt_sr + p];
            if (blk >= 0 && blk < NB) vfl[blk] = 0;
        }
    }
    phase_sync();
    int fcnt = 0, top = *top_p;
    // flush_collect (:141-191): per request, pages in order; a staged page
    // whose latch is clear is claimed into the flush list (while it has
    // room); every staged page that is not over the list's capacity is freed
    for (int r = 0; r < n_req; ++r) {
        const int s = sl[r], ql = qsl[r + 1] - qsl[r];
        if (s <= 0 || ql <= 0) continue;
        const int npc = min((s - ql) / page, bt_cols);
        if (npc <= 0) continue;
        const int ept = cdiv(npc, TB), a = tid * ept, b = min(a + ept, npc);
        const int* row = bt + (long)r * bt_sr;
        int n_new = 0;
        for (int p = a; p < b; ++p) {
            const int blk = row[p];
            if (blk < 0 || blk >= NB) continue;
            if (vbo[blk] >= 0 && vfl[blk] == 0) ++n_new;
        }
        int tot_new;
        const int base_new = block_scan_excl(n_new, wsum, &tot_new);
        int n_fre = 0, k = 0;
        for (int p = a; p < b; ++p) {
            const int blk = row[p];
            if (blk < 0 || blk >= NB || vbo[blk] < 0) continue;
            if (vfl[blk] == 0) n_fre += (fcnt + base_new + k++ < max_flush);
            else ++n_fre;
        }
        int tot_fre;
        const int base_fre = block_scan_excl(n_fre, wsum, &tot_fre);
        k = 0;
        int kf = 0;
        for (int p = a; p < b; ++p) {
            const int blk = row[p];
            if (blk < 0 || blk >= NB) continue;
            const int vb = vbo[blk];
            if (vb < 0) continue;
            if (vfl[blk] == 0) {
                const int idx = fcnt + base_new + k++;
                if (idx >= max_flush) continue;          // list full: stays staged
                flist[2 * idx] = blk;
                flist[2 * idx + 1] = vb;
                vfl[blk] = 1;
            }
            vbo[blk] = -1;                               // freed after the claim
            stack[top + base_fre + kf++] = vb;
        }
        fcnt = min(fcnt + tot_new, max_flush);
        top += tot_fre;
        phase_sync();
    }
    // valloc (:194-221): a staging block for every written page lacking one,
    // popped from the stack top in page order; underflow raises the latch
    for (int r = 0; r < n_req; ++r) {
        const int s = sl[r], ql = qsl[r + 1] - qsl[r];
        if (s <= 0 || ql <= 0) continue;
        const int p0 = (s - ql) / page, p1 = min((s - 1) / page, bt_cols - 1);
        const int np = p1 - p0 + 1;
        if (np <= 0) continue;
        const int ept = cdiv(np, TB), a = p0 + tid * ept, b = min(a + ept, p1 + 1);
        const int* row = bt + (long)r * bt_sr;
        int n_need = 0;
        for (int p = a; p < b; ++p) {
            const int blk = row[p];
            n_need += (blk >= 0 && blk < NB && vbo[blk] < 0);
        }
        int tot;
        const int base = block_scan_excl(n_need, wsum, &tot);
        int k = 0;
        for (int p = a; p < b; ++p) {
            const int blk = row[p];
            if (blk < 0 || blk >= NB || vbo[blk] >= 0) continue;
            const int idx = top - 1 - (base + k++);
            if (idx >= 0) vbo[blk] = stack[idx];
            else *overflow = 1;
        }
        top = max(top - tot, 0);
        phase_sync();
    }
    // vslot (:224-244): this step's token -> staging slot
    for (int r = 0; r < n_req; ++r) {
        const int s = sl[r], q0 = qsl[r], ql = qsl[r + 1] - q0;
        if (s <= 0 || ql <= 0) continue;
        for (int i = tid; i < ql; i += TB) {
            const int pos = s - ql + i, p = pos / page;
            const int blk = p < bt_cols ? bt[(long)r * bt_sr + p] : -1;
            const int vb = (blk >= 0 && blk < NB) ? vbo[blk] : -1;
            if (q0 + i < max_tokens)
                vslot[q0 + i] = (vb >= 0 && vb < NV) ? (long long)vb * page + pos % page : -1;
        }
    }
    if (tid == 0) {
        *top_p = top;
        *fcnt_p = fcnt;
    }
}

// flush copy (:247-277): grid (workgroups, layers); one wave per (entry, kv).
__global__ __launch_bounds__(256) void tier_flush_copy_kernel(
    const int* __restrict__ flist, const int* __restrict__ fcnt_p, int max_flush,
    const uint16_t* __restrict__ stg_v, const uint16_t* __restrict__ stg_k, long sl_, long sb,
    long st_, long sh, uint16_t* pool_v, uint16_t* pool_k, int8_t* pool_valid, int n_kv, int NB,
    int page, int D, int k_tier)
{
    const int l = blockIdx.y, lane = threadIdx.x & (kWave - 1);
    const int n = min(*fcnt_p, max_flush) * n_kv;
    const int rpt = D / 8;                               // 16-byte chunks per token row
    for (int e = blockIdx.x * 4 + (threadIdx.x >> 6); e < n; e += gridDim.x * 4) {
        const int i = e / n_kv, kv = e % n_kv;
        const int blk = flist[2 * i], vb = flist[2 * i + 1];
        const long dst = (((long)l * NB + blk) * n_kv + kv) * page * D;
        const long src = l * sl_ + vb * sb + kv * sh;
        for (int c = lane; c < page * rpt; c += kWave) {
            const int t = c / rpt, dd = (c % rpt) * 8;
            *reinterpret_cast<uint4*>(pool_v + dst + (long)t * D + dd) =
                *reinterpret_cast<const uint4*>(stg_v + src + t * st_ + dd);
            if (k_tier)
                *reinterpret_cast<uint4*>(pool_k + dst + (long)t * D + dd) =
                    *reinterpret_cast<const uint4*>(stg_k + src + t * st_ + dd);
        }
        if (lane == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            pool_valid[((long)l * n_kv + kv) * NB + blk] = 1;
        }
    }
}

// scatter (:57-82): grid (tokens); thread = (kv, 16-byte chunk).
__global__ __launch_bounds__(256) void tier_scatter_kernel(
    const uint16_t* __restrict__ val, long vt, long vh, const uint16_t* __restrict__ key, long kt,
    long kh, const long long* __restrict__ vslot, uint16_t* stg_v, uint16_t* stg_k, long sb,
    long st_, long sh, int n_kv, int D, int page, int NV, int k_tier)
{
    const int t = blockIdx.x;
    const long long vs = vslot[t];
    if (vs < 0 || vs >= (long long)NV * page) return;
    const long vb = (long)(vs / page), off = (long)(vs % page);
    const int rpt = D / 8;
    for (int c = threadIdx.x; c < n_kv * rpt; c += blockDim.x) {
        const int kv = c / rpt, dd = (c % rpt) * 8;
        const long dst = vb * sb + off * st_ + kv * sh + dd;
        *reinterpret_cast<uint4*>(stg_v + dst) =
            *reinterpret_cast<const uint4*>(val + (long)t * vt + kv * vh + dd);
        if (k_tier)
            *reinterpret_cast<uint4*>(stg_k + dst) =
                *reinterpret_cast<const uint4*>(key + (long)t * kt + kv * kh + dd);
    }
}

// ---------------------------------------------------------------------------
// residency plan (residency.py:51-145): one workgroup per kv head.
//
// A. hit / miss of every selected complete page, requests in order; a hit
//    touches its slot's clock; misses are compacted per (request, kv head) in
//    page-table order and numbered j in (request, page) order; each miss
//    records min(j) on page2slot[blk] (INT_MIN + j: below any slot and -1), so
//    the first occurrence of a block shared by several requests is known.
// B. unique misses ranked u = 0.. in j order (later occurrences: victim -1,
//    the reference's "installed earlier this pass").
// C. victims: the k = min(unique, eligible) smallest (clock, slot) keys of the
//    slots not touched this call, in ascending order (= the reference's
//    sequential argmin, each pick then touched).  Radix select of the rank's
//    clock (3 passes), the slot by a scan among that clock, candidates ranked
//    by counting in LDS, TP_KMAX ranks per round.
// D. unique miss u takes victim u: the old page loses its slot, the maps and
//    clock are installed, the fetch list entry (blk, slot) is written at u.
// The clock is per (layer, kv head): the reference's one global clock
// advances on every call of every layer, but a slot's clock is only compared
// with the clocks of the same (layer, kv head), so the eviction order is the
// same.
// ---------------------------------------------------------------------------
struct PlanArgs {
    const int* tab; long t_sr, t_sh; int t_cols;
    const int* cnt; long c_sr;
    const int* bt; long bt_sr; int bt_cols;
    const int* sl; int n_req;
    int *p2s, *s2p, *lru, *clock;
    int *miss, *miss_cnt, *vict, *flist, *fcnt, *overflow;
    int fcap, n_kv, NB, S, page;
};

// the R-th smallest (clock, slot) key among eligible slots (clock < clk)
__device__ unsigned long long kth_key(const int* LR, int S, int clk, int R, int* hist, int* wsum,
                                      int* sh)
{
    const int tid = threadIdx.x;
    unsigned int prefix = 0;
    int rem = R;
    const int shifts[3] = {21, 10, 0}, widths[3] = {11, 11, 10};
#pragma unroll
    for (int ps = 0; ps < 3; ++ps) {
        const int shift = shifts[ps], nb = 1 << widths[ps];
        for (int i = tid; i < TP_BINS; i += TB) hist[i] = 0;
        __syncthreads();
        const unsigned int hi_mask = ps == 0 ? 0u : (0xFFFFFFFFu << (shift + widths[ps]));
        for (int s = tid; s < S; s += TB) {
            const int v = ld_coh(LR + s);
            if (v < clk && ((unsigned)v & hi_mask) == prefix)
                atomicAdd(&hist[((unsigned)v >> shift) & (nb - 1)], 1);
        }
        __syncthreads();
        // bins (2 tid, 2 tid + 1): find the bin where the cumulative count passes rem
        const int c0 = hist[2 * tid], c1 = hist[2 * tid + 1];
        int tot;
        const int before = block_scan_excl(c0 + c1, wsum, &tot);
        if (rem >= before && rem < before + c0) { sh[0] = 2 * tid; sh[1] = before; }
        else if (rem >= before + c0 && rem < before + c0 + c1) { sh[0] = 2 * tid + 1; sh[1] = before + c0; }
        __syncthreads();
        prefix |= (unsigned)sh[0] << shift;
        rem -= sh[1];
        __syncthreads();
    }
    // the rem-th slot (in slot order) whose clock is exactly prefix
    int run = 0, slot = -1;
    for (int s0 = 0; s0 < S && slot < 0; s0 += TB) {
        const int s = s0 + tid;
        const int f = (s < S && ld_coh(LR + s) == (int)prefix) ? 1 : 0;
        int tot;
        const int pos = block_scan_excl(f, wsum, &tot);
        if (f && run + pos == rem) sh[2] = s;
        __syncthreads();
        if (run + tot > rem) slot = sh[2];
        run += tot;
        __syncthreads();
    }
    return ((unsigned long long)prefix << 32) | (unsigned)slot;
}

__global__ __launch_bounds__(TB) void tier_plan_kernel(PlanArgs a)
{
    __shared__ int wsum[TB_WAVES];
    __shared__ int hist[TP_BINS];
    __shared__ int sh[8];
    __shared__ unsigned long long ckey[TP_KMAX];
    const int kv = blockIdx.x, tid = threadIdx.x;
    int* P = a.p2s + (long)kv * a.NB;
    int* SP = a.s2p + (long)kv * a.S;
    int* LR = a.lru + (long)kv * a.S;
    int* FL = a.flist + (long)kv * a.fcap * 2;
    const int clk = a.clock[kv] + 1;
    // A
    int jbase = 0;
    for (int r = 0; r < a.n_req; ++r) {
        const int n = min(max(a.cnt[r * a.c_sr + kv], 0), a.t_cols);
        const int s = a.sl[r];
        const int* trow = a.tab + r * a.t_sr + kv * a.t_sh;
        int* mrow = a.miss + ((long)r * a.n_kv + kv) * a.t_cols;
        int moff = 0;
        for (int i0 = 0; i0 < n; i0 += TB) {
            const int i = i0 + tid;
            int blk = -1, miss = 0;
            if (i < n) {
                const int pt = trow[i];
                if (pt >= 0 && pt < a.bt_cols && (long)(pt + 1) * a.page <= s) {
                    blk = a.bt[r * a.bt_sr + pt];
                    if (blk >= 0 && blk < a.NB) {
                        const int slot = ld_coh(P + blk);
                        if (slot >= 0) { if (slot < a.S) st_coh(LR + slot, clk); }
                        else miss = 1;
                    }
                }
            }
            int tot;
            const int pos = block_scan_excl(miss, wsum, &tot);
            if (miss) {
                mrow[moff + pos] = blk;
                atomicMin(P + blk, INT_MIN + jbase + moff + pos);
            }
            moff += tot;
        }
        if (tid == 0) a.miss_cnt[r * a.n_kv + kv] = moff;
        jbase += moff;
    }
    phase_sync();
    // B
    int U = 0, j0 = 0;
    for (int r = 0; r < a.n_req; ++r) {
        const int m = a.miss_cnt[r * a.n_kv + kv];
        const int* mrow = a.miss + ((long)r * a.n_kv + kv) * a.t_cols;
        int* vrow = a.vict + ((long)r * a.n_kv + kv) * a.t_cols;
        for (int i0 = 0; i0 < m; i0 += TB) {
            const int i = i0 + tid;
            int first = 0;
            if (i < m) first = ld_coh(P + mrow[i]) == INT_MIN + j0 + i;
            int tot;
            const int pos = block_scan_excl(first, wsum, &tot);
            if (i < m) vrow[i] = first ? U + pos : -1;
            U += tot;
        }
        j0 += m;
    }
    // C (nothing to install: skip the slot scan)
    int n_elig = 0;
    if (U > 0) {
        int c = 0;
        for (int s = tid; s < a.S; s += TB) c += ld_coh(LR + s) < clk;
        int tot;
        block_scan_excl(c, wsum, &tot);
        n_elig = tot;
    }
    const int k = min(U, n_elig);
    unsigned long long t_prev = 0;
    bool have_prev = false;
    for (int base = 0; base < k; base += TP_KMAX) {
        const int kr = min(TP_KMAX, k - base);
        const unsigned long long t_hi = kth_key(LR, a.S, clk, base + kr - 1, hist, wsum, sh);
        if (tid == 0) sh[3] = 0;
        __syncthreads();
        for (int s = tid; s < a.S; s += TB) {
            const int v = ld_coh(LR + s);
            if (v >= clk) continue;
            const unsigned long long key = ((unsigned long long)(unsigned)v << 32) | (unsigned)s;
            if ((have_prev && key <= t_prev) || key > t_hi) continue;
            ckey[atomicAdd(&sh[3], 1)] = key;
        }
        __syncthreads();
        for (int i = tid; i < kr; i += TB) {
            const unsigned long long x = ckey[i];
            int rank = 0;
            for (int j = 0; j < kr; ++j) rank += ckey[j] < x;
            FL[2 * (base + rank) + 1] = (int)(x & 0xFFFFFFFFull);
        }
        t_prev = t_hi;
        have_prev = true;
        __syncthreads();
    }
    phase_sync();
    // D
    for (int r = 0; r < a.n_req; ++r) {
        const int m = a.miss_cnt[r * a.n_kv + kv];
        const int* mrow = a.miss + ((long)r * a.n_kv + kv) * a.t_cols;
        int* vrow = a.vict + ((long)r * a.n_kv + kv) * a.t_cols;
        for (int i = tid; i < m; i += TB) {
            const int u = vrow[i];
            if (u < 0) continue;
            const int blk = mrow[i];
            if (u < k) {
                const int slot = FL[2 * u + 1];
                const int old = ld_coh(SP + slot);
                if (old >= 0 && old < a.NB) st_coh(P + old, -1);
                st_coh(P + blk, slot);
                st_coh(SP + slot, blk);
                st_coh(LR + slot, clk);
                FL[2 * u] = blk;
                vrow[i] = slot;
            } else {
                st_coh(P + blk, -1);
                vrow[i] = -1;
                *a.overflow = 1;
            }
        }
    }
    if (tid == 0) {
        a.fcnt[kv] = k;
        a.clock[kv] = clk;
    }
}

// fetch (residency.py:216-268): grid (workgroups, kv heads); one wave per entry.
__global__ __launch_bounds__(256) void tier_fetch_kernel(
    const int* __restrict__ flist, const int* __restrict__ fcnt, int fcap, uint16_t* hot_v,
    uint16_t* hot_k, uint16_t* pool_v, uint16_t* pool_k, const uint16_t* __restrict__ stg_v,
    const uint16_t* __restrict__ stg_k, long sb, long st_, long sh, const int* __restrict__ vbo,
    int8_t* pool_valid, int layer, int n_kv, int NB, int S, int NV, int page, int D, int k_tier)
{
    const int kv = blockIdx.y, lane = threadIdx.x & (kWave - 1);
    const int n = min(fcnt[kv], fcap);
    const long pe = (long)page * D;
    const int rpt = D / 8;
    for (int u = blockIdx.x * 4 + (threadIdx.x >> 6); u < n; u += gridDim.x * 4) {
        const int blk = flist[((long)kv * fcap + u) * 2], slot = flist[((long)kv * fcap + u) * 2 + 1];
        if (blk < 0 || blk >= NB || slot < 0 || slot >= S) continue;
        int8_t* vld = pool_valid + (long)kv * NB + blk;
        const long hot_off = ((long)kv * S + slot) * pe;
        const long pool_off = (((long)layer * NB + blk) * n_kv + kv) * pe;
        const int vb = vbo[blk];
        if (*vld > 0 || vb < 0 || vb >= NV) {
            wave_copy(hot_v + hot_off, pool_v + pool_off, pe, lane);
            if (k_tier) wave_copy(hot_k + hot_off, pool_k + pool_off, pe, lane);
            continue;
        }
        const long src = (long)vb * sb + (long)kv * sh;
        for (int c = lane; c < page * rpt; c += kWave) {
            const int t = c / rpt, dd = (c % rpt) * 8;
            const uint4 x = *reinterpret_cast<const uint4*>(stg_v + src + t * st_ + dd);
            *reinterpret_cast<uint4*>(hot_v + hot_off + (long)t * D + dd) = x;
            *reinterpret_cast<uint4*>(pool_v + pool_off + (long)t * D + dd) = x;
            if (k_tier) {
                const uint4 y = *reinterpret_cast<const uint4*>(stg_k + src + t * st_ + dd);
                *reinterpret_cast<uint4*>(hot_k + hot_off + (long)t * D + dd) = y;
                *reinterpret_cast<uint4*>(pool_k + pool_off + (long)t * D + dd) = y;
            }
        }
        if (lane == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            *vld = 1;
        }
    }
}

bool tier_geom_ok(int head_dim, int page) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
           (page == 16 || page == 32 || page == 64);
}

}  // namespace
}  // namespace locks

using namespace locks;

extern "C" int32_t locks_tier_invalidate(const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                                         const int32_t* seq_lens, const int32_t* query_start_loc,
                                         int32_t n_req, int32_t* page2slot, int32_t* slot2page,
                                         int8_t* pool_valid, int32_t num_layers, int32_t n_kv,
                                         int32_t num_blocks, int32_t hot_slots, int32_t page, void* stream)
{
    LOCKS_REQUIRE(block_table && seq_lens && query_start_loc && page2slot && slot2page && pool_valid,
                  "locks_tier_invalidate: null pointer argument");
    LOCKS_REQUIRE(n_req >= 0 && num_layers >= 1 && n_kv >= 1 && num_blocks >= 1 && hot_slots >= 1 &&
                  bt_cols >= 1 && page >= 1, "locks_tier_invalidate: bad geometry");
    if (n_req == 0) return 0;
    hipLaunchKernelGGL(tier_invalidate_kernel, dim3(n_req), dim3(256), 0, (hipStream_t)stream,
                       block_table, (long)bt_stride, bt_cols, seq_lens, query_start_loc, page2slot,
                       slot2page, pool_valid, num_layers, n_kv, num_blocks, hot_slots, page);
    return check_launch("tier_invalidate_kernel");
}

extern "C" int32_t locks_tier_stage_begin(const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                                          const int32_t* seq_lens, const int32_t* query_start_loc,
                                          int32_t n_req, int32_t* vbo, int32_t* v_flushed,
                                          int32_t* free_stack, int32_t* free_top, int32_t* flush_list,
                                          int32_t* flush_cnt, int32_t max_flush, int64_t* v_slot_mapping,
                                          int32_t max_tokens, int32_t* overflow, int32_t num_blocks,
                                          int32_t stage_blocks, int32_t page, void* stream)
{
    LOCKS_REQUIRE(block_table && seq_lens && query_start_loc && vbo && v_flushed && free_stack &&
                  free_top && flush_list && flush_cnt && v_slot_mapping && overflow,
                  "locks_tier_stage_begin: null pointer argument");
    LOCKS_REQUIRE(n_req >= 0 && bt_cols >= 1 && max_flush >= 1 && max_tokens >= 1 && num_blocks >= 1 &&
                  stage_blocks >= 1 && page >= 1, "locks_tier_stage_begin: bad geometry");
    hipLaunchKernelGGL(tier_stage_begin_kernel, dim3(1), dim3(TB), 0, (hipStream_t)stream, block_table,
                       (long)bt_stride, bt_cols, seq_lens, query_start_loc, n_req, vbo, v_flushed,
                       free_stack, free_top, flush_list, flush_cnt, max_flush,
                       reinterpret_cast<long long*>(v_slot_mapping), max_tokens, overflow, num_blocks,
                       stage_blocks, page);
    return check_launch("tier_stage_begin_kernel");
}

extern "C" int32_t locks_tier_flush_copy(const int32_t* flush_list, const int32_t* flush_cnt,
                                         int32_t max_flush, const uint16_t* stage_v, const uint16_t* stage_k,
                                         int64_t stage_stride_layer, int64_t stage_stride_block,
                                         int64_t stage_stride_tok, int64_t stage_stride_head,
                                         uint16_t* pool_v, uint16_t* pool_k, int8_t* pool_valid,
                                         int32_t num_layers, int32_t n_kv, int32_t num_blocks, int32_t page,
                                         int32_t head_dim, int32_t k_tier, void* stream)
{
    LOCKS_REQUIRE(flush_list && flush_cnt && stage_v && pool_v && pool_valid,
                  "locks_tier_flush_copy: null pointer argument");
    LOCKS_REQUIRE(!k_tier || (stage_k && pool_k), "locks_tier_flush_copy: k_tier needs the K pools");
    LOCKS_REQUIRE(tier_geom_ok(head_dim, page) && num_layers >= 1 && n_kv >= 1 && num_blocks >= 1 &&
                  max_flush >= 1, "locks_tier_flush_copy: bad geometry (head_dim %d, page %d)", head_dim, page);
    LOCKS_REQUIRE(stage_stride_layer % 8 == 0 && stage_stride_block % 8 == 0 && stage_stride_tok % 8 == 0 &&
                  stage_stride_head % 8 == 0, "locks_tier_flush_copy: staging strides must be multiples of 8");
    const int wg = min(cdiv(max_flush * n_kv, 4), 256);
    hipLaunchKernelGGL(tier_flush_copy_kernel, dim3(wg, num_layers), dim3(256), 0, (hipStream_t)stream,
                       flush_list, flush_cnt, max_flush, stage_v, stage_k, (long)stage_stride_layer,
                       (long)stage_stride_block, (long)stage_stride_tok, (long)stage_stride_head, pool_v,
                       pool_k, pool_valid, n_kv, num_blocks, page, head_dim, k_tier ? 1 : 0);
    return check_launch("tier_flush_copy_kernel");
}

extern "C" int32_t locks_tier_scatter(const uint16_t* value, int64_t v_stride_tok, int64_t v_stride_head,
                                      const uint16_t* key, int64_t k_stride_tok, int64_t k_stride_head,
                                      int32_t n_tokens, const int64_t* v_slot_mapping, uint16_t* stage_v,
                                      uint16_t* stage_k, int64_t stage_stride_block, int64_t stage_stride_tok,
                                      int64_t stage_stride_head, int32_t n_kv, int32_t head_dim, int32_t page,
                                      int32_t stage_blocks, int32_t k_tier, void* stream)
{
    LOCKS_REQUIRE(value && v_slot_mapping && stage_v, "locks_tier_scatter: null pointer argument");
    LOCKS_REQUIRE(!k_tier || (key && stage_k), "locks_tier_scatter: k_tier needs key and the K staging pool");
    LOCKS_REQUIRE(tier_geom_ok(head_dim, page) && n_kv >= 1 && n_kv * head_dim / 8 <= 1024 &&
                  n_tokens >= 0 && stage_blocks >= 1,
                  "locks_tier_scatter: bad geometry (n_kv %d, head_dim %d, page %d)", n_kv, head_dim, page);
    LOCKS_REQUIRE(v_stride_tok % 8 == 0 && v_stride_head % 8 == 0 && (!k_tier || (k_stride_tok % 8 == 0 &&
                  k_stride_head % 8 == 0)) && stage_stride_block % 8 == 0 && stage_stride_tok % 8 == 0 &&
                  stage_stride_head % 8 == 0, "locks_tier_scatter: strides must be multiples of 8 elements");
    if (n_tokens == 0) return 0;
    hipLaunchKernelGGL(tier_scatter_kernel, dim3(n_tokens), dim3(256), 0, (hipStream_t)stream, value,
                       (long)v_stride_tok, (long)v_stride_head, key, (long)k_stride_tok, (long)k_stride_head,
                       reinterpret_cast<const long long*>(v_slot_mapping), stage_v, stage_k,
                       (long)stage_stride_block, (long)stage_stride_tok, (long)stage_stride_head, n_kv,
                       head_dim, page, stage_blocks, k_tier ? 1 : 0);
    return check_launch("tier_scatter_kernel");
}

extern "C" int32_t locks_tier_plan(const int32_t* page_table, int64_t pt_stride_req, int64_t pt_stride_head,
                                   int32_t pt_cols, const int32_t* page_cnt, int64_t cnt_stride,
                                   const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
                                   const int32_t* seq_lens, int32_t n_req, int32_t* page2slot,
                                   int32_t* slot2page, int32_t* lru, int32_t* clock, int32_t* miss_pages,
                                   int32_t* miss_cnt, int32_t* victims, int32_t* fetch_list,
                                   int32_t* fetch_cnt, int32_t fetch_cap, int32_t* overflow, int32_t n_kv,
                                   int32_t num_blocks, int32_t hot_slots, int32_t page, void* stream)
{
    LOCKS_REQUIRE(page_table && page_cnt && block_table && seq_lens && page2slot && slot2page && lru &&
                  clock && miss_pages && miss_cnt && victims && fetch_list && fetch_cnt && overflow,
                  "locks_tier_plan: null pointer argument");
    LOCKS_REQUIRE(n_req >= 0 && n_kv >= 1 && num_blocks >= 1 && hot_slots >= 1 && pt_cols >= 1 &&
                  bt_cols >= 1 && page >= 1, "locks_tier_plan: bad geometry");
    LOCKS_REQUIRE(num_blocks < (1 << 30) && (long)n_req * pt_cols < (1L << 30),
                  "locks_tier_plan: num_blocks / n_req x pages too large");
    LOCKS_REQUIRE((long)fetch_cap >= (long)n_req * pt_cols,
                  "locks_tier_plan: fetch_cap %d < n_req %d x pt_cols %d", fetch_cap, n_req, pt_cols);
    PlanArgs a{page_table, (long)pt_stride_req, (long)pt_stride_head, pt_cols, page_cnt, (long)cnt_stride,
               block_table, (long)bt_stride, bt_cols, seq_lens, n_req, page2slot, slot2page, lru, clock,
               miss_pages, miss_cnt, victims, fetch_list, fetch_cnt, overflow, fetch_cap, n_kv,
               num_blocks, hot_slots, page};
    hipLaunchKernelGGL(tier_plan_kernel, dim3(n_kv), dim3(TB), 0, (hipStream_t)stream, a);
    return check_launch("tier_plan_kernel");
}

extern "C" int32_t locks_tier_fetch(const int32_t* fetch_list, const int32_t* fetch_cnt, int32_t fetch_cap,
                                    uint16_t* hot_v, uint16_t* hot_k, uint16_t* pool_v, uint16_t* pool_k,
                                    const uint16_t* stage_v, const uint16_t* stage_k,
                                    int64_t stage_stride_block, int64_t stage_stride_tok,
                                    int64_t stage_stride_head, const int32_t* vbo, int8_t* pool_valid,
                                    int32_t layer, int32_t num_layers, int32_t n_kv, int32_t num_blocks,
                                    int32_t hot_slots, int32_t stage_blocks, int32_t page, int32_t head_dim,
                                    int32_t k_tier, void* stream)
{
    LOCKS_REQUIRE(fetch_list && fetch_cnt && hot_v && pool_v && stage_v && vbo && pool_valid,
                  "locks_tier_fetch: null pointer argument");
    LOCKS_REQUIRE(!k_tier || (hot_k && pool_k && stage_k), "locks_tier_fetch: k_tier needs the K buffers");
    LOCKS_REQUIRE(tier_geom_ok(head_dim, page) && n_kv >= 1 && num_blocks >= 1 && hot_slots >= 1 &&
                  stage_blocks >= 1 && fetch_cap >= 1,
                  "locks_tier_fetch: bad geometry (head_dim %d, page %d)", head_dim, page);
    LOCKS_REQUIRE(layer >= 0 && layer < num_layers, "locks_tier_fetch: layer %d outside [0, %d)", layer,
                  num_layers);
    LOCKS_REQUIRE(stage_stride_block % 8 == 0 && stage_stride_tok % 8 == 0 && stage_stride_head % 8 == 0,
                  "locks_tier_fetch: staging strides must be multiples of 8 elements");
    // 8 workgroups (32 waves) per kv head: enough page copies in flight to
    // fill the host link on a cold step, few enough to launch fast when
    // every page hits
    const int wg = min(cdiv(fetch_cap, 4), 8);
    hipLaunchKernelGGL(tier_fetch_kernel, dim3(wg, n_kv), dim3(256), 0, (hipStream_t)stream, fetch_list,
                       fetch_cnt, fetch_cap, hot_v, hot_k, pool_v, pool_k, stage_v, stage_k,
                       (long)stage_stride_block, (long)stage_stride_tok, (long)stage_stride_head, vbo,
                       pool_valid, layer, n_kv, num_blocks, hot_slots, stage_blocks, page, head_dim,
                       k_tier ? 1 : 0);
    return check_launch("tier_fetch_kernel");
}
