// Split-K sparse paged decode + LSE merge for gfx950.
//
// Semantics (reference: attention/decode.py:209-322, attention/merge.py:105-152):
//   per (request r, kv head kh, split sp):
//     pps = max(cdiv(cnt, SPLIT), PPS_MIN); pages [sp*pps, min(sp*pps+pps, cnt))
//     of page_table[r][kh] (logical ids, ascending); block = block_table[r][pt];
//     K/V tile = kv[block, :, kh, :] (16 tokens x d); token pt*16+t is masked
//     when >= seq_len; online softmax over the split's tokens for all G heads
//     of the group; partials m, l (G) and acc (G, d) in fp32.  Inactive splits
//     store nothing.
//   merge: n_act = cdiv(cnt, pps); w = (l > 0) ? exp(m - max m) : 0;
//     out = sum w*acc / sum w*l  (0 when the denominator is 0).
//
// MI355X mapping: one wave per split.  Per 16-token page the wave issues
// 8 x 16-byte loads per lane (K rows for the QK operand, V rows for the PV
// operand), prefetching the next page while it computes the current one.
//   * S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (A = K tile: token rows; B = the
//     GQA group's q rows, zero padded to 16) -- bf16 products, fp32 sum, like
//     the reference's bf16 tl.dot.  Each lane ends with 4 tokens of one head.
//     The k-slot -> d map is chosen so each K load reads 64 contiguous bytes
//     per token row.
//   * online softmax per head: 4-token in-lane max + 2 cross-row shuffles.
//   * O^T += V^T P^T on v_mfma_f32_16x16x16f16 with fp16 P and fp16 V (the
//     reference's fp16 P.V with fp32 accumulation).  The V operand needs no
//     transpose: the output d-index of MFMA block `blk`, row i is 8*i + blk,
//     so each lane's four 16-byte V row loads ARE its A operand.  The softmax
//     rescale is a per-lane scalar because O^T keeps one head per lane.
#include "locks_common.h"
#include "locks_hip.h"

#include <algorithm>
#include <mutex>

namespace locks {

constexpr int DC_PG = 16;
constexpr int DC_WAVES = 4;
constexpr int DC_BLK = DC_WAVES * kWave;
typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(3))) const uint8_t* lds_u8_ptr;
typedef int v2i __attribute__((ext_vector_type(2)));
constexpr int MAX_SPLIT = 512;
constexpr int DENSE_NST = 2;           // page stages per wave of the dense comparator
// K/V DMA cache policy: NT (non-temporal: every page is read once) measured
// 5.58 -> 5.97 TB/s for the dense comparator at 1M (SC1 did not help); the
// sparse decode measured the same step time with and without it.
constexpr int CPOL_NT = 2;

__device__ __forceinline__ uint32_t bf16_word(const uint4& w, int e) {
    const uint32_t x = (e >> 1) == 0 ? w.x : (e >> 1) == 1 ? w.y : (e >> 1) == 2 ? w.z : w.w;
    return (e & 1) ? (x >> 16) : (x & 0xFFFFu);
}

// Device-coherent partials for the fused decode: 16-byte buffer loads and
// stores with the SC1 cache policy (the gfx950 encoding of device-scope
// relaxed atomics) -- written by one workgroup, read by another of the same
// launch after an arrival count, with no cache write-back or invalidate.
constexpr int CPOL_SC1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7fffffff, 0x00020000);
}
template <bool COHERENT>
__device__ __forceinline__ float4 ld_part4(const float* base, long idx) {
    if constexpr (COHERENT) {
        const v4i v = __builtin_amdgcn_raw_buffer_load_b128(part_rsrc(base), (int)(idx * 4), 0, CPOL_SC1);
        return __builtin_bit_cast(float4, v);
    } else {
        return *reinterpret_cast<const float4*>(base + idx);
    }
}
template <bool COHERENT>
__device__ __forceinline__ float ld_part(const float* base, long idx) {
    if constexpr (COHERENT)
        return __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(part_rsrc(base), (int)(idx * 4), 0, CPOL_SC1));
    else return base[idx];
}

// Merge the first n_act split partials of row rk into out (one workgroup,
// DC_BLK threads).  w_s, l_s: >= MAX_SPLIT * 16 floats of LDS each.
// Work split: the row's G * D / 4 float4 output columns ("items") times
// `grp` split streams fill the workgroup (at most two items per thread).
// Every thread issues the loads of its first MR_PF splits' partials before
// anything waits, together with the m / l loads, so a row of up to
// grp * MR_PF splits costs one memory round trip; the streams are summed in
// LDS at the end.
constexpr int MR_PF = 16;
template <bool COHERENT = false, int D = 128>
__device__ void merge_row(const float* __restrict__ m_part, const float* __restrict__ l_part,
                          const float* __restrict__ acc_part, long rk, int r, int kh, int n_act,
                          int G, int split, void* __restrict__ out, long o_sr, long o_sh,
                          int out_f32, float* w_s, float* l_s, float* lt_s) {
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr int NWV = DC_BLK / kWave;
    constexpr int CPR = D / 4;                          // float4 columns per head
    const int n_items = G * CPR;
    const int grp = n_items >= DC_BLK ? 1 : DC_BLK / n_items;
    const int stream = n_items >= DC_BLK ? 0 : tid / n_items;
    const int item0 = n_items >= DC_BLK ? tid : tid % n_items;
    const bool two = n_items > DC_BLK;                  // G > 8: items tid and tid + DC_BLK
    const bool live = stream < grp;                     // threads past grp * n_items idle
    // partial index of (item, split s): ((rk * split + s) * G + g) * CPR + c
    //   = rk * split * n_items + s * n_items + item
    const long rowbase = rk * split * (long)n_items;
    float4 pre[2][MR_PF];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int item = min(item0 + it * DC_BLK, n_items - 1);
#pragma unroll
        for (int k = 0; k < MR_PF; ++k) {
            const int sidx = min(stream + k * grp, split - 1);
            pre[it][k] = (it == 0 || two)
                ? ld_part4<COHERENT>(acc_part, (rowbase + (long)sidx * n_items + item) * 4)
                : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    // every (split, head) m and l, up to 4 per thread in flight, then the
    // per-head max / weights / denominator from LDS
    float* m_s = w_s;                                   // [s * 16 + g], reused for the weights
    const int nml = n_act * G;
    for (int i0 = tid; i0 < nml; i0 += 4 * DC_BLK) {
        float mv[4], lv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = min(i0 + j * DC_BLK, nml - 1);
            const int sidx = i / G, g = i - sidx * G;
            const long src = (rk * split + sidx) * G + g;
            mv[j] = ld_part<COHERENT>(m_part, src);
            lv[j] = ld_part<COHERENT>(l_part, src);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = i0 + j * DC_BLK;
            if (i < nml) {
                const int sidx = i / G, g = i - sidx * G;
                m_s[sidx * 16 + g] = mv[j];
                l_s[sidx * 16 + g] = lv[j];
            }
        }
    }
    __syncthreads();
    for (int g = wave; g < G; g += NWV) {
        float mm = -INFINITY;
        for (int sidx = lane; sidx < n_act; sidx += kWave)
            if (l_s[sidx * 16 + g] > 0.f) mm = fmaxf(mm, m_s[sidx * 16 + g]);
        mm = wave_max(mm);
        float lt = 0.f;
        for (int sidx = lane; sidx < n_act; sidx += kWave) {
            const float l = l_s[sidx * 16 + g];
            const float w = (l > 0.f) ? __expf(m_s[sidx * 16 + g] - mm) : 0.f;
            m_s[sidx * 16 + g] = w;                     // this lane read it last
            lt += l * w;
        }
        lt = wave_sum(lt);
        if (lane == 0) lt_s[g] = lt;
    }
    __syncthreads();
    float4 accs[2];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int item = min(item0 + it * DC_BLK, n_items - 1);
        const int g = item / CPR;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int k = 0; k < MR_PF; ++k) {
            const int sidx = stream + k * grp;
            if (sidx < n_act) {
                const float w = w_s[sidx * 16 + g];
                const float4 a = pre[it][k];
                acc.x += w * a.x; acc.y += w * a.y; acc.z += w * a.z; acc.w += w * a.w;
            }
        }
        // splits past the prefetched ones (rows of more than grp * MR_PF
        // splits): batches of 8 loads, then their FMAs
        for (int k0 = MR_PF; stream + k0 * grp < n_act; k0 += 8) {
            float4 b[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int sidx = min(stream + (k0 + k) * grp, split - 1);
                b[k] = ld_part4<COHERENT>(acc_part, (rowbase + (long)sidx * n_items + item) * 4);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int sidx = stream + (k0 + k) * grp;
                if (sidx < n_act) {
                    const float w = w_s[sidx * 16 + g];
                    acc.x += w * b[k].x; acc.y += w * b[k].y; acc.z += w * b[k].z; acc.w += w * b[k].w;
                }
            }
        }
        accs[it] = acc;
    }
    float4* red = reinterpret_cast<float4*>(l_s);        // [stream][item], after the weights
    if (grp > 1) {
        if (live) red[stream * n_items + item0] = accs[0];
        __syncthreads();
    }
    if (stream != 0 || !live) return;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        if (it == 1 && !two) break;
        const int item = item0 + it * DC_BLK;
        if (item >= n_items) break;
        float4 acc = accs[it];
        for (int sg = 1; sg < grp; ++sg) {
            const float4 a = red[sg * n_items + item];
            acc.x += a.x; acc.y += a.y; acc.z += a.z; acc.w += a.w;
        }
        const int g = item / CPR, d4 = (item % CPR) * 4;
        const float lt = lt_s[g];
        const float inv = (lt > 0.f) ? 1.f / lt : 0.f;
        const float o[4] = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
        const long oi = (long)r * o_sr + (long)(kh * G + g) * o_sh + d4;
        if (out_f32) {
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + oi) =
                make_float4(o[0], o[1], o[2], o[3]);
        } else {
            uint16_t* ob = reinterpret_cast<uint16_t*>(out) + oi;
#pragma unroll
            for (int e = 0; e < 4; ++e) ob[e] = f32_to_bf16(o[e]);
        }
    }
}

// Per-head_dim constants of the split kernel.  A step is 16 tokens of one
// (page, kv head): K 16 x D and V 16 x D bf16 in one LDS stage.
template <int D>
struct DcGeom {
    static_assert(D == 64 || D == 128 || D == 256, "head_dim 64, 128 or 256");
    static constexpr int KS = D / 32;                   // QK k-slots: one 16-byte DMA per lane each
    static constexpr int DPL = D / 16;                  // V columns per lane (PV output blocks)
    static constexpr int VI = D == 64 ? 2 : 4 * (DPL / 8);   // V DMA instructions per step
    static constexpr int NI = KS + VI;                  // DMA instructions per step
    static constexpr int KBYTES = 16 * D * 2;
    static constexpr int STEP_BYTES = 2 * KBYTES;
};

constexpr int vm_wait_imm(int n) {                       // s_waitcnt vmcnt(n) lgkmcnt(0)
    return 0x0070 | (n & 15) | ((n >> 4) << 14);
}
template <int NI, int NST>
__device__ __forceinline__ void wait_vm_steps(int ahead) {
    // vmcnt(NI * ahead): the steps issued after the one to consume
    switch (ahead) {
        case 0: __builtin_amdgcn_s_waitcnt(vm_wait_imm(0)); break;
        case 1: __builtin_amdgcn_s_waitcnt(vm_wait_imm(NI)); break;
        case 2: if constexpr (NST > 2) __builtin_amdgcn_s_waitcnt(vm_wait_imm(2 * NI)); break;
        default: if constexpr (NST > 3) __builtin_amdgcn_s_waitcnt(vm_wait_imm(3 * NI)); break;
    }
}

// One workgroup = 4 waves per split; wave w takes the split's 16-token steps
// s0+w, s0+w+4, ... (a page of PG tokens is PG/16 consecutive steps).
// Steps are DMA'd into per-wave LDS stages with global_load_lds_dwordx4 in
// the lane order the MFMA operands need, so in-flight steps cost no VGPRs;
// NST stages form a ring (NST - 1 steps in flight while one is consumed).
// The 4 wave states are then merged in LDS into the split's partial.
// DENSE: every page of the row in logical order (page count from seq_len,
// no page table) -- the dense full-KV comparator.  KVPOL: cache policy bits
// of the K/V DMA.  pg_sh: log2(page / 16).
// DRAM-tier V source (reference attention/decode_cuda.py:178-222, the mem
// tier's per-(page, kv head) pointer select): a complete page whose (kv
// head, block) holds a hot slot reads the hot buffer (n_kv, S, page, d);
// else a staged block (vbo >= 0) reads the staging pool at its strides; else
// the pinned host pool (L, NB, n_kv, page, d), device-visible.  K follows
// the same select when k_tier (mem-kv), else stays in the paged cache.
struct TierSrc {
    const uint16_t* hotv; const uint16_t* stgv; const uint16_t* poolv;
    const uint16_t* hotk; const uint16_t* stgk; const uint16_t* poolk;
    const int* p2s; const int* vbo;
    long svb, svt, svh, S, NV;
    int lidx, k_tier;
};

template <bool FUSED, bool DENSE = false, int NST = 2, int KVPOL = 0, int D = 128, bool TIER = false>
__global__ __launch_bounds__(DC_BLK) void decode_split_kernel(
    const uint16_t* __restrict__ q, long q_sr, long q_sh,
    const uint16_t* __restrict__ kc, long k_sb, long k_st, long k_sh,
    const uint16_t* __restrict__ vc, long v_sb, long v_st, long v_sh,
    int NB, const int* __restrict__ bt, long bt_sr, int bt_cols,
    const int* __restrict__ ptab, long pt_sr, long pt_sh, int pt_cols,
    const int* __restrict__ pcnt, long cnt_sr, const int* __restrict__ seq_lens,
    float* __restrict__ m_part, float* __restrict__ l_part, float* __restrict__ acc_part,
    int G, int split, int pps_min, float sm_scale, int pg_sh,
    int* __restrict__ counters, void* __restrict__ out, long o_sr, long o_sh, int out_f32,
    const TierSrc tier)
{
    using GM = DcGeom<D>;
    static_assert(!(TIER && (FUSED || DENSE)), "the tier source serves the split kernel");
    constexpr int KS = GM::KS, DPL = GM::DPL, NI = GM::NI, KB = GM::KBYTES, SB = GM::STEP_BYTES;
    const int sp = blockIdx.x, kh = blockIdx.y, r = blockIdx.z;
    const int n_kv = gridDim.y;
    const long rk = (long)r * n_kv + kh;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    static_assert(NST >= 2 && NST <= 4, "page stages per wave");
    static_assert(!(FUSED && DENSE), "the dense comparator merges in its own launch");
    const int PG = DC_PG << pg_sh, smask = (1 << pg_sh) - 1;
    const int* prow = ptab + (long)r * pt_sr + (long)kh * pt_sh;
    // This wave's first page ids assuming pps == pps_min (the usual sparse
    // case), loaded together with the page count instead of after it.
    const int js = ((sp * pps_min) << pg_sh) + wave + DC_WAVES * lane;
    int pt_spec = 0, cnt;
    if constexpr (DENSE) {
        cnt = min(cdiv(seq_lens[r], PG), bt_cols);
    } else {
        pt_spec = ((js >> pg_sh) < pt_cols) ? prow[js >> pg_sh] : 0;
        cnt = min(pcnt[(long)r * cnt_sr + kh], pt_cols);
    }
    // gridDim.x = the launched split count (<= split, the buffers' stride)
    const int nsplit = gridDim.x;
    const int pps = max(cdiv(cnt, nsplit), pps_min);
    const int j0 = sp * pps;
    if constexpr (FUSED) {
        if (cnt <= 0) {                           // nothing selected: the output row is 0
            if (sp == 0)
                for (int i = threadIdx.x; i < G * D; i += DC_BLK) {
                    const long oi = (long)r * o_sr + (long)(kh * G + i / D) * o_sh + i % D;
                    if (out_f32) static_cast<float*>(out)[oi] = 0.f;
                    else static_cast<uint16_t*>(out)[oi] = 0;
                }
            return;
        }
    }
    if (j0 >= cnt) return;                        // inactive split: no store
    const int j1 = min(j0 + pps, cnt);
    const int s0 = j0 << pg_sh, s1 = j1 << pg_sh; // this split's 16-token steps

    const int c16 = lane & 15, kg = lane >> 4;
    const int seq_len = seq_lens[r];

    // NST step stages per wave (stage 0 in stA, the others in stB), later
    // reused for the merges (the fused merge needs MAX_SPLIT x 16 floats in each)
    constexpr int MIN_REGION = FUSED ? MAX_SPLIT * 16 * 4 : 0;
    constexpr int A_BYTES = DC_WAVES * SB > MIN_REGION ? DC_WAVES * SB : MIN_REGION;
    constexpr int B_BYTES = (NST - 1) * DC_WAVES * SB > MIN_REGION ? (NST - 1) * DC_WAVES * SB : MIN_REGION;
    static_assert(A_BYTES >= DC_WAVES * 16 * D * 4, "wave-merge buffer fits stage A");
    __shared__ __attribute__((aligned(16))) uint8_t stA[A_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t stB[B_BYTES];
    __shared__ float wm[DC_WAVES][16], wl[DC_WAVES][16];
    auto stage = [&](int i) -> uint8_t* {
        return i == 0 ? stA + wave * SB : stB + ((i - 1) * DC_WAVES + wave) * SB;
    };

    // B operand of QK, k-slot (kg, s) <-> d = 32*s + 8*kg + 0..7
    v8bf qb[KS];
    {
        const uint16_t* qp = q + (long)r * q_sr + (long)(kh * G + c16) * q_sh + 8 * kg;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            uint4 w = make_uint4(0u, 0u, 0u, 0u);
            if (c16 < G) w = *reinterpret_cast<const uint4*>(qp + 32 * s);
            qb[s] = __builtin_bit_cast(v8bf, w);
        }
    }

    // Page and block ids of up to 64 steps of this wave are fetched up front
    // (lane i holds step i), so no dependent id load sits behind a stage's
    // DMA in the in-order vmcnt queue.
    int ptv = 0, blkv = 0, slotv = -1, vbov = -1;
    auto fetch_ids = [&](int jb, bool spec) {
        const int jj = jb + DC_WAVES * lane;
        ptv = 0;
        blkv = 0;
        if (jj < s1) {
            if constexpr (DENSE) ptv = jj >> pg_sh;
            else ptv = spec ? pt_spec : prow[jj >> pg_sh];
            const int ptc = min(max(ptv, 0), bt_cols - 1);
            blkv = min(max(bt[(long)r * bt_sr + ptc], 0), NB - 1);
            if constexpr (TIER) {                 // the tier's keys of (kv head, block)
                slotv = tier.p2s[(long)kh * NB + blkv];
                vbov = tier.vbo[blkv];
            }
        }
    };
    // DMA step s of the current id batch (16 tokens from token 16 * sub of
    // its page) into stage `st`:
    //   K slot i (< KS) = K[t = lane&15][32 i + 8 kg ..], 1 KB per slot;
    //   V (D >= 128) slot (i, hh) = V[4 kg + i][DPL (lane&15) + 8 hh ..];
    //   V (D == 64) in natural row order (8 lanes per 128-byte row).
    auto issue = [&](int s, int sub, uint8_t* st) -> int {
        const int pt = __builtin_amdgcn_readlane(ptv, s);
        const int blk = __builtin_amdgcn_readlane(blkv, s);
        const long t0 = (long)sub * 16;
        const uint16_t* kpage = kc + (long)blk * k_sb + (long)kh * k_sh;
        const uint16_t* vpage = vc + (long)blk * v_sb + (long)kh * v_sh;
        long kst = k_st, vst = v_st;
        if constexpr (TIER) {
            // one wave-uniform source per (page, kv head)
            const int slot = __builtin_amdgcn_readlane(slotv, s);
            const int vbs = __builtin_amdgcn_readlane(vbov, s);
            const bool complete = (long)(pt + 1) * PG <= (long)seq_len;
            const bool hot = complete && slot >= 0 && slot < tier.S;   // out-of-range keys: the pool
            const bool stg = !hot && vbs >= 0 && vbs < tier.NV;
            const long pe = (long)PG * D;
            const long hot_off = ((long)kh * tier.S + (hot ? slot : 0)) * pe;
            const long stg_off = (long)(stg ? vbs : 0) * tier.svb + (long)kh * tier.svh;
            const long pin_off = (((long)tier.lidx * NB + blk) * n_kv + kh) * pe;
            vpage = hot ? tier.hotv + hot_off : stg ? tier.stgv + stg_off : tier.poolv + pin_off;
            vst = stg ? tier.svt : (long)D;
            if (tier.k_tier) {
                kpage = hot ? tier.hotk + hot_off : stg ? tier.stgk + stg_off : tier.poolk + pin_off;
                kst = vst;
            }
        }
        const uint16_t* kp = kpage + (t0 + c16) * kst + 8 * kg;
#pragma unroll
        for (int i = 0; i < KS; ++i)
            __builtin_amdgcn_global_load_lds(kp + 32 * i, (lds_ptr)(st + i * 1024), 16, 0, KVPOL);
        const uint16_t* vb = vpage + t0 * vst;
        if constexpr (D == 64) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
                __builtin_amdgcn_global_load_lds(vb + (long)(8 * i + (lane >> 3)) * vst + 8 * (lane & 7),
                                                 (lds_ptr)(st + KB + i * 1024), 16, 0, KVPOL);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int hh = 0; hh < DPL / 8; ++hh)
                    __builtin_amdgcn_global_load_lds(vb + (long)(4 * kg + i) * vst + DPL * c16 + 8 * hh,
                                                     (lds_ptr)(st + KB + (i * (DPL / 8) + hh) * 1024), 16, 0, KVPOL);
        }
        return pt;
    };

    float m = -INFINITY, lsum = 0.f;
    v4f o[DPL];
#pragma unroll
    for (int b = 0; b < DPL; ++b) o[b] = v4f{0.f, 0.f, 0.f, 0.f};

    auto consume = [&](const uint8_t* st, int pt, int sub) {
        // The stage is read with ds_read in inline asm: the compiler cannot
        // tell these reads from the other stages' DMA still in flight and
        // would otherwise wait for every outstanding load (vmcnt(0)) here.
        // The caller has already waited for this stage's own DMA.  One asm
        // block per head_dim, so nothing uses a result before the wait.
        v4i kr[KS];
        uint32_t vw[4][DPL / 2];                     // V row v: DPL bf16 columns
        const uint32_t sbase = (uint32_t)(uintptr_t)(lds_u8_ptr)(st);
        const uint32_t la = sbase + lane * 16;
        if constexpr (D == 64) {
            v2i v64[4];
            const uint32_t lv = sbase + KB + kg * 512 + c16 * 8;   // row 4 kg, columns 4 c16 ..
            asm volatile(
                "ds_read_b128 %0, %6\n\t"
                "ds_read_b128 %1, %6 offset:1024\n\t"
                "ds_read_b64 %2, %7\n\t"
                "ds_read_b64 %3, %7 offset:128\n\t"
                "ds_read_b64 %4, %7 offset:256\n\t"
                "ds_read_b64 %5, %7 offset:384\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=v"(kr[0]), "=v"(kr[1]), "=v"(v64[0]), "=v"(v64[1]), "=v"(v64[2]), "=v"(v64[3])
                : "v"(la), "v"(lv));
#pragma unroll
            for (int v = 0; v < 4; ++v) { vw[v][0] = (uint32_t)v64[v][0]; vw[v][1] = (uint32_t)v64[v][1]; }
        } else if constexpr (D == 128) {
            v4i vr[4];
            asm volatile(
                "ds_read_b128 %0, %8\n\t"
                "ds_read_b128 %1, %8 offset:1024\n\t"
                "ds_read_b128 %2, %8 offset:2048\n\t"
                "ds_read_b128 %3, %8 offset:3072\n\t"
                "ds_read_b128 %4, %8 offset:4096\n\t"
                "ds_read_b128 %5, %8 offset:5120\n\t"
                "ds_read_b128 %6, %8 offset:6144\n\t"
                "ds_read_b128 %7, %8 offset:7168\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=v"(kr[0]), "=v"(kr[1]), "=v"(kr[2]), "=v"(kr[3]),
                  "=v"(vr[0]), "=v"(vr[1]), "=v"(vr[2]), "=v"(vr[3])
                : "v"(la));
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int e = 0; e < 4; ++e) vw[v][e] = (uint32_t)vr[v][e];
        } else {
            v4i vr[8];
            const uint32_t la2 = la + 8192;          // the second 8 KB of the stage
            asm volatile(
                "ds_read_b128 %0, %16\n\t"
                "ds_read_b128 %1, %16 offset:1024\n\t"
                "ds_read_b128 %2, %16 offset:2048\n\t"
                "ds_read_b128 %3, %16 offset:3072\n\t"
                "ds_read_b128 %4, %16 offset:4096\n\t"
                "ds_read_b128 %5, %16 offset:5120\n\t"
                "ds_read_b128 %6, %16 offset:6144\n\t"
                "ds_read_b128 %7, %16 offset:7168\n\t"
                "ds_read_b128 %8, %17\n\t"
                "ds_read_b128 %9, %17 offset:1024\n\t"
                "ds_read_b128 %10, %17 offset:2048\n\t"
                "ds_read_b128 %11, %17 offset:3072\n\t"
                "ds_read_b128 %12, %17 offset:4096\n\t"
                "ds_read_b128 %13, %17 offset:5120\n\t"
                "ds_read_b128 %14, %17 offset:6144\n\t"
                "ds_read_b128 %15, %17 offset:7168\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=v"(kr[0]), "=v"(kr[1]), "=v"(kr[2]), "=v"(kr[3]),
                  "=v"(kr[4]), "=v"(kr[5]), "=v"(kr[6]), "=v"(kr[7]),
                  "=v"(vr[0]), "=v"(vr[1]), "=v"(vr[2]), "=v"(vr[3]),
                  "=v"(vr[4]), "=v"(vr[5]), "=v"(vr[6]), "=v"(vr[7])
                : "v"(la), "v"(la2));
            // slot (v, hh) = vr[2 v + hh]: columns 16 c16 + 8 hh ..
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int e = 0; e < 8; ++e) vw[v][e] = (uint32_t)vr[2 * v + (e >> 2)][e & 3];
        }
        // ---- S^T[t][g] = K[t] . q[g] ------------------------------------
        v4f s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < KS; ++i)
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, kr[i]), qb[i], s, 0, 0, 0);
        const int pos0 = pt * PG + sub * 16 + 4 * kg;
        float sv[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) sv[v] = (pos0 + v < seq_len) ? s[v] * sm_scale : -INFINITY;
        // ---- online softmax (head = lane column) ------------------------
        float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        mx = xor32_max(xor16_max(mx));
        const float m_new = fmaxf(m, mx);
        const float m_ref = (m_new == -INFINITY) ? 0.f : m_new;   // fully masked so far
        const float alpha = __expf(m - m_ref);
        float p[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) p[v] = __expf(sv[v] - m_ref);
        lsum = lsum * alpha + (p[0] + p[1] + p[2] + p[3]);
        m = m_new;
        const v4h pb = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
        // ---- O^T[d][g] += V^T P^T: block b holds d = DPL * row + b --------
#pragma unroll
        for (int b = 0; b < DPL; ++b) {
            v4h a;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const uint32_t w = vw[v][b >> 1];
                a[v] = (_Float16)bf16_to_f32((uint16_t)((b & 1) ? (w >> 16) : (w & 0xFFFFu)));
            }
            o[b] = o[b] * alpha;
            o[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pb, o[b], 0, 0, 0);
        }
    };

    for (int jb = s0 + wave; jb < s1; jb += DC_WAVES * kWave) {
        fetch_ids(jb, pps == pps_min && jb == s0 + wave);
        __builtin_amdgcn_s_waitcnt(0x0070);   // ids (and q) resident before any DMA
        const int ns = min(kWave, cdiv(s1 - jb, DC_WAVES));   // steps of this batch
        auto sub_of = [&](int s) { return (jb + DC_WAVES * s) & smask; };
        // ring of NST stages: step s + NST - 1 is issued before step s is
        // consumed, so up to NST - 1 steps stream while one is scored
#pragma unroll
        for (int i = 0; i < NST - 1; ++i)
            if (i < ns) issue(i, sub_of(i), stage(i));
        int si = 0, ii = NST - 1;
        for (int s = 0; s < ns; ++s) {
            if (s + NST - 1 < ns) issue(s + NST - 1, sub_of(s + NST - 1), stage(ii));
            wait_vm_steps<NI, NST>(min(NST - 1, ns - 1 - s));
            __builtin_amdgcn_wave_barrier();
            consume(stage(si), __builtin_amdgcn_readlane(ptv, s), sub_of(s));
            __builtin_amdgcn_wave_barrier();
            si = (si + 1 == NST) ? 0 : si + 1;
            ii = (ii + 1 == NST) ? 0 : ii + 1;
        }
    }
    lsum = xor32_sum(xor16_sum(lsum));

    // ---- merge the 4 wave states of this split in LDS --------------------
    __syncthreads();                              // every stage consumed
    float* red = reinterpret_cast<float*>(stA);   // [wave][g][d]
    if (kg == 0) { wm[wave][c16] = m; wl[wave][c16] = lsum; }
    {
        // lane (g = c16, kg), row v of block b <-> d = DPL * (4 kg + v) + b
        float* ow = red + (wave * 16 + c16) * D + DPL * 4 * kg;
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int j = 0; j < DPL / 4; ++j)
                *reinterpret_cast<float4*>(ow + DPL * v + 4 * j) =
                    make_float4(o[4 * j][v], o[4 * j + 1][v], o[4 * j + 2][v], o[4 * j + 3][v]);
    }
    __syncthreads();
    const long base = (rk * split + sp) * G;
    for (int i = tid; i < G * (D / 4); i += DC_BLK) {
        const int g = i / (D / 4), d = (i % (D / 4)) * 4;
        float M = wm[0][g];
#pragma unroll
        for (int w = 1; w < DC_WAVES; ++w) M = fmaxf(M, wm[w][g]);
        const float Mr = (M == -INFINITY) ? 0.f : M;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        float l = 0.f;
#pragma unroll
        for (int w = 0; w < DC_WAVES; ++w) {
            const float e = __expf(wm[w][g] - Mr);
            const float4 x = *reinterpret_cast<const float4*>(red + (w * 16 + g) * D + d);
            acc.x += e * x.x; acc.y += e * x.y; acc.z += e * x.z; acc.w += e * x.w;
            l += e * wl[w][g];
        }
        if constexpr (FUSED) {
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, acc), part_rsrc(acc_part),
                                                   (int)(((base + g) * D + d) * 4), 0, CPOL_SC1);
            if (d == 0) {
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(M), part_rsrc(m_part), (int)((base + g) * 4), 0, CPOL_SC1);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(l), part_rsrc(l_part), (int)((base + g) * 4), 0, CPOL_SC1);
            }
        } else {
            *reinterpret_cast<float4*>(acc_part + (base + g) * D + d) = acc;
            if (d == 0) { m_part[base + g] = M; l_part[base + g] = l; }
        }
    }
    if constexpr (FUSED) {
        // The last of the row's active splits to finish merges them all.
        // Protocol (every access to the partials is device-coherent: SC1
        // stores and loads, the gfx950 encoding of agent-scope relaxed
        // atomic stores / loads, which bypass the per-XCD L2):
        //   1. each wave waits for its own SC1 stores to be acknowledged
        //      (vmcnt(0): the data is at the device coherence point);
        //   2. a workgroup release fence + barrier orders those waits before
        //      thread 0's arrival (it also keeps the compiler from moving any
        //      store past the barrier);
        //   3. an agent-scope atomic counts arrivals; the workgroup that sees
        //      the last one acquires (agent-scope fence after the barrier)
        //      and reads the partials with SC1 loads, which cannot hit a
        //      stale L2 line.
        // Each row's counter sits in its own 256-B block: with the counters
        // of all rows packed in one cache line, every arrival of the launch
        // serialised on that line (measured +1.7 us per launch at Llama
        // 128K: 256 arrivals).
        // An agent-scope release on every arrival would add an L2 write-back
        // (buffer_wbl2) to every workgroup: measured +8 us per layer at Llama
        // 128K (step 1.35 -> 1.62 ms, with the acquire side in every
        // workgroup too), for data that never goes through the L2 here.
        __shared__ int last_s;
        __shared__ float lt_s[16];
        __builtin_amdgcn_s_waitcnt(0x0070);           // vmcnt(0): SC1 stores acknowledged
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __syncthreads();
        const int n_act = min(cdiv(cnt, pps), nsplit);
        if (tid == 0) {
            const int old = __hip_atomic_fetch_add(counters + rk * LOCKS_DECODE_COUNTER_STRIDE, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_s = (old == n_act - 1);
        }
        __syncthreads();
        if (!last_s) return;
        // the reader side under the memory model: an agent-scope acquire in
        // the row's last workgroup only (one per row, so its L2 invalidate
        // is not paid by every split)
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        if (tid == 0) __hip_atomic_store(counters + rk * LOCKS_DECODE_COUNTER_STRIDE, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        merge_row<true, D>(m_part, l_part, acc_part, rk, r, kh, n_act, G, split, out, o_sr, o_sh,
                           out_f32, reinterpret_cast<float*>(stA), reinterpret_cast<float*>(stB), lt_s);
    }
}

// LSE merge of one (request, kv head, query head) row of split partials,
// one workgroup per head: D / 4 float4 columns x 1024 / D split streams, so a row is
// merged by G workgroups (G CUs' memory parallelism) instead of one.  The
// page count is page_cnt (clamped to pt_cols, as the split kernel) or, with
// pcnt == nullptr, the dense one (every page of the row).
constexpr int MH_BLK = 256;
constexpr int MH_PF = 8;                   // partials prefetched per thread
template <int D>
__global__ __launch_bounds__(MH_BLK) void decode_merge_heads_kernel(
    const float* __restrict__ m_part, const float* __restrict__ l_part,
    const float* __restrict__ acc_part, const int* __restrict__ pcnt, long cnt_sr, int pt_cols,
    const int* __restrict__ seq_lens, int bt_cols,
    void* __restrict__ out, long o_sr, long o_sh, int out_f32, int G, int split, int nsplit,
    int pps_min, int pg)
{
    constexpr int MH_COLS = D / 4, MH_STREAMS = MH_BLK / MH_COLS;   // float4 columns x split streams
    const int g = blockIdx.x, kh = blockIdx.y, r = blockIdx.z;
    const int n_kv = gridDim.y;
    const long rk = (long)r * n_kv + kh;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = tid % MH_COLS, strm = tid / MH_COLS;
    // Every load is issued before anything waits: the page count, this
    // thread's (split, m, l) and its first MH_PF partial columns, at split
    // indices clamped into the buffers (entries past the active count are
    // masked below, never combined), so the merge costs one round trip.
    const int cnt_raw = pcnt ? pcnt[(long)r * cnt_sr + kh] : seq_lens[r];
    // (clamped to the launched splits, not the buffer's: rows past them were
    // never written this call, and reading them only doubled the traffic)
    float4 pre[MH_PF];
#pragma unroll
    for (int k = 0; k < MH_PF; ++k) {
        const int sidx = min(strm + k * MH_STREAMS, nsplit - 1);
        pre[k] = *reinterpret_cast<const float4*>(acc_part + ((rk * split + sidx) * G + g) * D + col * 4);
    }
    const long ml0 = (rk * split + min(tid, nsplit - 1)) * G + g;
    const float m0 = m_part[ml0], l0 = l_part[ml0];
    const int cnt = pcnt ? min(cnt_raw, pt_cols) : min(cdiv(cnt_raw, pg), bt_cols);
    const int pps = max(cdiv(cnt, nsplit), pps_min);
    const int n_act = cnt > 0 ? min(cdiv(cnt, pps), nsplit) : 0;
    __shared__ float w_s[MAX_SPLIT];
    __shared__ float red[MH_BLK / kWave];
    __shared__ float4 part[MH_STREAMS][MH_COLS];
    // head max over the splits that hold mass
    const bool has0 = tid < n_act && l0 > 0.f;
    float mm = has0 ? m0 : -INFINITY;
    for (int s = tid + MH_BLK; s < n_act; s += MH_BLK) {   // rows of more than MH_BLK splits
        const long i = (rk * split + s) * G + g;
        if (l_part[i] > 0.f) mm = fmaxf(mm, m_part[i]);
    }
    mm = wave_max(mm);
    if (lane == 0) red[wave] = mm;
    lds_barrier();
    mm = red[0];
#pragma unroll
    for (int w = 1; w < MH_BLK / kWave; ++w) mm = fmaxf(mm, red[w]);
    lds_barrier();
    const float w0 = has0 ? __expf(m0 - mm) : 0.f;
    if (tid < n_act) w_s[tid] = w0;
    float lt = has0 ? l0 * w0 : 0.f;
    for (int s = tid + MH_BLK; s < n_act; s += MH_BLK) {
        const long i = (rk * split + s) * G + g;
        const float l = l_part[i];
        const float w = (l > 0.f) ? __expf(m_part[i] - mm) : 0.f;
        w_s[s] = w;
        lt += l * w;
    }
    lt = wave_sum(lt);
    if (lane == 0) red[wave] = lt;
    lds_barrier();
    lt = 0.f;
#pragma unroll
    for (int w = 0; w < MH_BLK / kWave; ++w) lt += red[w];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    // weights of the prefetched partials: every LDS read issued before the
    // first use (a guarded read per partial was one LDS round trip each);
    // partials past the active count are left out by selects
    float wk[MH_PF];
#pragma unroll
    for (int k = 0; k < MH_PF; ++k) wk[k] = w_s[min(strm + k * MH_STREAMS, MAX_SPLIT - 1)];
#pragma unroll
    for (int k = 0; k < MH_PF; ++k) {          // selects, not branches (stale rows may hold NaN)
        const bool on = strm + k * MH_STREAMS < n_act;
        const float w = wk[k];
        acc.x = on ? acc.x + w * pre[k].x : acc.x;
        acc.y = on ? acc.y + w * pre[k].y : acc.y;
        acc.z = on ? acc.z + w * pre[k].z : acc.z;
        acc.w = on ? acc.w + w * pre[k].w : acc.w;
    }
#pragma unroll 4
    for (int s = strm + MH_PF * MH_STREAMS; s < n_act; s += MH_STREAMS) {
        const float w = w_s[s];
        const float4 a = *reinterpret_cast<const float4*>(acc_part + ((rk * split + s) * G + g) * D + col * 4);
        acc.x += w * a.x; acc.y += w * a.y; acc.z += w * a.z; acc.w += w * a.w;
    }
    part[strm][col] = acc;
    lds_barrier();
    if (tid < MH_COLS) {
        float4 t = part[0][col];
#pragma unroll
        for (int k = 1; k < MH_STREAMS; ++k) {
            const float4 a = part[k][col];
            t.x += a.x; t.y += a.y; t.z += a.z; t.w += a.w;
        }
        const float inv = (lt > 0.f) ? 1.f / lt : 0.f;
        const float o[4] = {t.x * inv, t.y * inv, t.z * inv, t.w * inv};
        const long oi = (long)r * o_sr + (long)(kh * G + g) * o_sh + col * 4;
        if (out_f32) {
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + oi) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
            uint16_t* ob = reinterpret_cast<uint16_t*>(out) + oi;
#pragma unroll
            for (int e = 0; e < 4; ++e) ob[e] = f32_to_bf16(o[e]);
        }
    }
}

// ---- no-allocation variant of the fused decode ----------------------------
// Scratch of locks_decode_fused_noalloc: the arrival counters (first 256-B
// aligned block), then the m, l and acc split partials.  One copy per GPU,
// held until the process ends; every call on a GPU shares it.
static __device__ __align__(256) uint8_t scratch[LOCKS_NOALLOC_SCRATCH_BYTES];

__global__ __launch_bounds__(256) void zero_i32_kernel(int* __restrict__ p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

}  // namespace locks

using namespace locks;

// Splits launched: enough for max_cnt pages at pps_min pages each (max_cnt
// is the caller's bound on page_cnt; 0 = none), at most `split`.  The
// kernels derive pps from the launched count, so a count above the bound is
// still decoded in full, in fewer, longer splits.
static int launched_splits(int split, int pps_min, int max_cnt) {
    return max_cnt > 0 ? std::min(split, std::max(1, cdiv(max_cnt, pps_min))) : split;
}

// head_dim in {64, 128, 256}, page in {16, 32, 64} (the reference's geometry
// domain, rki4_state.py:295-324); pg_sh = log2(page / 16)
static bool dc_geometry(int head_dim, int page, int* pg_sh) {
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return false;
    if (page != 16 && page != 32 && page != 64) return false;
    *pg_sh = page == 16 ? 0 : page == 32 ? 1 : 2;
    return true;
}
// launch KERNEL<..., D> for the runtime head_dim
#define DC_BY_D(HD, LAUNCH_D)                               \
    do {                                                     \
        if ((HD) == 64) { LAUNCH_D(64); }                    \
        else if ((HD) == 128) { LAUNCH_D(128); }             \
        else { LAUNCH_D(256); }                              \
    } while (0)

static int32_t decode_splitk_impl(
    const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
    const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok, int64_t k_stride_head,
    const uint16_t* v_cache, int64_t v_stride_block, int64_t v_stride_tok, int64_t v_stride_head,
    int32_t num_blocks, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
    const int32_t* page_table, int64_t pt_stride_req, int64_t pt_stride_head, int32_t pt_cols,
    const int32_t* page_cnt, int64_t cnt_stride, const int32_t* seq_lens,
    float* m_part, float* l_part, float* acc_part,
    int32_t n_req, int32_t n_kv, int32_t G, int32_t head_dim, int32_t page,
    int32_t split, int32_t pps_min, int32_t max_cnt, float sm_scale, void* stream,
    const locks_tier_src* ts)
{
    int pg_sh = 0;
    LOCKS_REQUIRE(dc_geometry(head_dim, page, &pg_sh),
                  "locks_decode_splitk: head_dim %d / page %d outside {64,128,256} x {16,32,64}", head_dim, page);
    LOCKS_REQUIRE(G >= 1 && G <= 16, "locks_decode_splitk: G=%d outside [1, 16]", G);
    LOCKS_REQUIRE(split >= 1 && split <= MAX_SPLIT, "locks_decode_splitk: split %d outside [1, %d]", split, MAX_SPLIT);
    LOCKS_REQUIRE(pps_min >= 1, "locks_decode_splitk: pps_min %d < 1", pps_min);
    LOCKS_REQUIRE(num_blocks >= 1 && bt_cols >= 1 && pt_cols >= 1, "locks_decode_splitk: empty geometry");
    LOCKS_REQUIRE(k_stride_tok % 8 == 0 && v_stride_tok % 8 == 0 && k_stride_block % 8 == 0 &&
                  v_stride_block % 8 == 0 && k_stride_head % 8 == 0 && v_stride_head % 8 == 0 &&
                  q_stride_req % 8 == 0 && q_stride_head % 8 == 0,
                  "locks_decode_splitk: q/K/V strides must be multiples of 8 elements (16-byte loads)");
    LOCKS_REQUIRE(q && k_cache && v_cache && block_table && page_table && page_cnt && seq_lens &&
                  m_part && l_part && acc_part, "locks_decode_splitk: null pointer argument");
    TierSrc tier{};
    if (ts) {
        LOCKS_REQUIRE(ts->hot_v && ts->stage_v && ts->pool_v && ts->page2slot && ts->vbo,
                      "locks_decode_splitk_tier: null tier pointer");
        LOCKS_REQUIRE(!ts->k_tier || (ts->hot_k && ts->stage_k && ts->pool_k),
                      "locks_decode_splitk_tier: k_tier needs the K hot / staging / pool pointers");
        LOCKS_REQUIRE(ts->num_blocks == num_blocks,
                      "locks_decode_splitk_tier: tier num_blocks %d != cache num_blocks %d", ts->num_blocks, num_blocks);
        LOCKS_REQUIRE(ts->hot_slots >= 0 && ts->stage_blocks >= 0,
                      "locks_decode_splitk_tier: hot_slots %d / stage_blocks %d < 0",
                      ts->hot_slots, ts->stage_blocks);
        LOCKS_REQUIRE(ts->n_kv == n_kv && ts->page == page && ts->head_dim == head_dim,
                      "locks_decode_splitk_tier: tier laid out for n_kv %d / page %d / head_dim %d, "
                      "call has %d / %d / %d", ts->n_kv, ts->page, ts->head_dim, n_kv, page, head_dim);
        LOCKS_REQUIRE(ts->layer >= 0 && ts->layer < ts->num_layers,
                      "locks_decode_splitk_tier: layer %d outside the pool's [0, %d)",
                      ts->layer, ts->num_layers);
        LOCKS_REQUIRE(ts->stage_stride_block % 8 == 0 && ts->stage_stride_tok % 8 == 0 &&
                      ts->stage_stride_head % 8 == 0,
                      "locks_decode_splitk_tier: staging strides must be multiples of 8 elements");
        tier = TierSrc{ts->hot_v, ts->stage_v, ts->pool_v, ts->hot_k, ts->stage_k, ts->pool_k,
                       ts->page2slot, ts->vbo, (long)ts->stage_stride_block, (long)ts->stage_stride_tok,
                       (long)ts->stage_stride_head, (long)ts->hot_slots, (long)ts->stage_blocks, ts->layer,
                       ts->k_tier ? 1 : 0};
    }
    if (n_req == 0) return 0;
#define LAUNCH_D(DV)                                                                                   \
    if (ts) hipLaunchKernelGGL((decode_split_kernel<false, false, 2, 0, DV, true>),                   \
                       dim3(launched_splits(split, pps_min, max_cnt), n_kv, n_req), dim3(DC_BLK), 0,    \
                       (hipStream_t)stream, q, (long)q_stride_req, (long)q_stride_head, k_cache,       \
                       (long)k_stride_block, (long)k_stride_tok, (long)k_stride_head, v_cache,         \
                       (long)v_stride_block, (long)v_stride_tok, (long)v_stride_head, num_blocks,      \
                       block_table, (long)bt_stride, bt_cols, page_table, (long)pt_stride_req,         \
                       (long)pt_stride_head, pt_cols, page_cnt, (long)cnt_stride, seq_lens,            \
                       m_part, l_part, acc_part, G, split, pps_min, sm_scale, pg_sh,                   \
                       nullptr, nullptr, 0L, 0L, 0, tier);                                              \
    else hipLaunchKernelGGL((decode_split_kernel<false, false, 2, 0, DV>),                             \
                       dim3(launched_splits(split, pps_min, max_cnt), n_kv, n_req), dim3(DC_BLK), 0,    \
                       (hipStream_t)stream, q, (long)q_stride_req, (long)q_stride_head, k_cache,       \
                       (long)k_stride_block, (long)k_stride_tok, (long)k_stride_head, v_cache,         \
                       (long)v_stride_block, (long)v_stride_tok, (long)v_stride_head, num_blocks,      \
                       block_table, (long)bt_stride, bt_cols, page_table, (long)pt_stride_req,         \
                       (long)pt_stride_head, pt_cols, page_cnt, (long)cnt_stride, seq_lens,            \
                       m_part, l_part, acc_part, G, split, pps_min, sm_scale, pg_sh,                   \
                       nullptr, nullptr, 0L, 0L, 0, TierSrc{})
    DC_BY_D(head_dim, LAUNCH_D);
#undef LAUNCH_D
    return check_launch("decode_split_kernel");
}

extern "C" int32_t locks_decode_splitk(
    const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
    const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok, int64_t k_stride_head,
    const uint16_t* v_cache, int64_t v_stride_block, int64_t v_stride_tok, int64_t v_stride_head,
    int32_t num_blocks, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
    const int32_t* page_table, int64_t pt_stride_req, int64_t pt_stride_head, int32_t pt_cols,
    const int32_t* page_cnt, int64_t cnt_stride, const int32_t* seq_lens,
    float* m_part, float* l_part, float* acc_part,
    int32_t n_req, int32_t n_kv, int32_t G, int32_t head_dim, int32_t page,
    int32_t split, int32_t pps_min, int32_t max_cnt, float sm_scale, void* stream)
{
    return decode_splitk_impl(q, q_stride_req, q_stride_head, k_cache, k_stride_block, k_stride_tok,
                              k_stride_head, v_cache, v_stride_block, v_stride_tok, v_stride_head,
                              num_blocks, block_table, bt_stride, bt_cols, page_table, pt_stride_req,
                              pt_stride_head, pt_cols, page_cnt, cnt_stride, seq_lens, m_part, l_part,
                              acc_part, n_req, n_kv, G, head_dim, page, split, pps_min, max_cnt,
                              sm_scale, stream, nullptr);
}

extern "C" int32_t locks_decode_splitk_tier(
    const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
    const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok, int64_t k_stride_head,
    const uint16_t* v_cache, int64_t v_stride_block, int64_t v_stride_tok, int64_t v_stride_head,
    int32_t num_blocks, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
    const int32_t* page_table, int64_t pt_stride_req, int64_t pt_stride_head, int32_t pt_cols,
    const int32_t* page_cnt, int64_t cnt_stride, const int32_t* seq_lens,
    float* m_part, float* l_part, float* acc_part,
    int32_t n_req, int32_t n_kv, int32_t G, int32_t head_dim, int32_t page,
    int32_t split, int32_t pps_min, int32_t max_cnt, float sm_scale,
    const locks_tier_src* tier, void* stream)
{
    LOCKS_REQUIRE(tier, "locks_decode_splitk_tier: null tier");
    return decode_splitk_impl(q, q_stride_req, q_stride_head, k_cache, k_stride_block, k_stride_tok,
                              k_stride_head, v_cache, v_stride_block, v_stride_tok, v_stride_head,
                              num_blocks, block_table, bt_stride, bt_cols, page_table, pt_stride_req,
                              pt_stride_head, pt_cols, page_cnt, cnt_stride, seq_lens, m_part, l_part,
                              acc_part, n_req, n_kv, G, head_dim, page, split, pps_min, max_cnt,
                              sm_scale, stream, tier);
}

extern "C" int32_t locks_host_device_pointer(void* host, void** dev)
{
    LOCKS_REQUIRE(host && dev, "locks_host_device_pointer: null pointer argument");
    const hipError_t e = hipHostGetDevicePointer(dev, host, 0);
    LOCKS_REQUIRE(e == hipSuccess && *dev, "locks_host_device_pointer: %p is not pinned host memory (%s)",
                  host, hipGetErrorString(e));
    return 0;
}

extern "C" int32_t locks_decode_fused(
    const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
    const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok, int64_t k_stride_head,
    const uint16_t* v_cache, int64_t v_stride_block, int64_t v_stride_tok, int64_t v_stride_head,
    int32_t num_blocks, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
    const int32_t* page_table, int64_t pt_stride_req, int64_t pt_stride_head, int32_t pt_cols,
    const int32_t* page_cnt, int64_t cnt_stride, const int32_t* seq_lens,
    float* m_part, float* l_part, float* acc_part, int32_t* counters,
    void* out, int64_t out_stride_req, int64_t out_stride_head, int32_t out_is_f32,
    int32_t n_req, int32_t n_kv, int32_t G, int32_t head_dim, int32_t page,
    int32_t split, int32_t pps_min, int32_t max_cnt, float sm_scale, void* stream)
{
    int pg_sh = 0;
    LOCKS_REQUIRE(dc_geometry(head_dim, page, &pg_sh),
                  "locks_decode_fused: head_dim %d / page %d outside {64,128,256} x {16,32,64}", head_dim, page);
    LOCKS_REQUIRE(G >= 1 && G <= 16, "locks_decode_fused: G=%d outside [1, 16]", G);
    LOCKS_REQUIRE(split >= 1 && split <= MAX_SPLIT, "locks_decode_fused: split %d outside [1, %d]", split, MAX_SPLIT);
    LOCKS_REQUIRE(pps_min >= 1, "locks_decode_fused: pps_min %d < 1", pps_min);
    LOCKS_REQUIRE(num_blocks >= 1 && bt_cols >= 1 && pt_cols >= 1, "locks_decode_fused: empty geometry");
    LOCKS_REQUIRE(k_stride_tok % 8 == 0 && v_stride_tok % 8 == 0 && k_stride_block % 8 == 0 &&
                  v_stride_block % 8 == 0 && k_stride_head % 8 == 0 && v_stride_head % 8 == 0 &&
                  q_stride_req % 8 == 0 && q_stride_head % 8 == 0,
                  "locks_decode_fused: q/K/V strides must be multiples of 8 elements (16-byte loads)");
    LOCKS_REQUIRE(out_stride_req % 4 == 0 && out_stride_head % 4 == 0,
                  "locks_decode_fused: out strides must be multiples of 4 elements");
    LOCKS_REQUIRE((int64_t)n_req * n_kv * split * G * head_dim * 4 < 0x7fffffffLL,
                  "locks_decode_fused: partials exceed 2 GiB");
    LOCKS_REQUIRE(q && k_cache && v_cache && block_table && page_table && page_cnt && seq_lens &&
                  m_part && l_part && acc_part && counters && out, "locks_decode_fused: null pointer argument");
    if (n_req == 0) return 0;
#define LAUNCH_D(DV)                                                                                   \
    hipLaunchKernelGGL((decode_split_kernel<true, false, 2, 0, DV>),                                   \
                       dim3(launched_splits(split, pps_min, max_cnt), n_kv, n_req), dim3(DC_BLK), 0,    \
                       (hipStream_t)stream, q, (long)q_stride_req, (long)q_stride_head, k_cache,       \
                       (long)k_stride_block, (long)k_stride_tok, (long)k_stride_head, v_cache,         \
                       (long)v_stride_block, (long)v_stride_tok, (long)v_stride_head, num_blocks,      \
                       block_table, (long)bt_stride, bt_cols, page_table, (long)pt_stride_req,         \
                       (long)pt_stride_head, pt_cols, page_cnt, (long)cnt_stride, seq_lens,            \
                       m_part, l_part, acc_part, G, split, pps_min, sm_scale, pg_sh,                   \
                       counters, out, (long)out_stride_req, (long)out_stride_head, out_is_f32, TierSrc{})
    DC_BY_D(head_dim, LAUNCH_D);
#undef LAUNCH_D
    return check_launch("decode_split_kernel<fused>");
}

extern "C" int32_t locks_decode_merge(
    const float* m_part, const float* l_part, const float* acc_part,
    const int32_t* page_cnt, int64_t cnt_stride, int32_t pt_cols, void* out, int64_t out_stride_req,
    int64_t out_stride_head, int32_t out_is_f32, int32_t n_req, int32_t n_kv, int32_t G,
    int32_t head_dim, int32_t split, int32_t pps_min, int32_t max_cnt, void* stream)
{
    LOCKS_REQUIRE(pt_cols >= 1, "locks_decode_merge: pt_cols %d < 1", pt_cols);
    LOCKS_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
                  "locks_decode_merge: head_dim %d outside {64, 128, 256}", head_dim);
    LOCKS_REQUIRE(G >= 1 && G <= 16, "locks_decode_merge: G=%d outside [1, 16]", G);
    LOCKS_REQUIRE(split >= 1 && split <= MAX_SPLIT, "locks_decode_merge: split %d outside [1, %d]", split, MAX_SPLIT);
    LOCKS_REQUIRE(pps_min >= 1, "locks_decode_merge: pps_min %d < 1", pps_min);
    LOCKS_REQUIRE(m_part && l_part && acc_part && page_cnt && out, "locks_decode_merge: null pointer argument");
    LOCKS_REQUIRE(out_stride_req % 4 == 0 && out_stride_head % 4 == 0,
                  "locks_decode_merge: out strides must be multiples of 4 elements");
    if (n_req == 0) return 0;
#define LAUNCH_D(DV)                                                                                \
    hipLaunchKernelGGL(decode_merge_heads_kernel<DV>, dim3(G, n_kv, n_req), dim3(MH_BLK), 0,        \
                       (hipStream_t)stream, m_part, l_part, acc_part, page_cnt, (long)cnt_stride,   \
                       pt_cols, nullptr, 1, out, (long)out_stride_req, (long)out_stride_head,       \
                       out_is_f32, G, split, launched_splits(split, pps_min, max_cnt), pps_min, 16)
    DC_BY_D(head_dim, LAUNCH_D);
#undef LAUNCH_D
    return check_launch("decode_merge_kernel");
}


extern "C" int32_t locks_decode_dense(
    const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
    const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok, int64_t k_stride_head,
    const uint16_t* v_cache, int64_t v_stride_block, int64_t v_stride_tok, int64_t v_stride_head,
    int32_t num_blocks, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
    const int32_t* seq_lens, float* m_part, float* l_part, float* acc_part,
    void* out, int64_t out_stride_req, int64_t out_stride_head, int32_t out_is_f32,
    int32_t n_req, int32_t n_kv, int32_t G, int32_t head_dim, int32_t page,
    int32_t split, float sm_scale, void* stream)
{
    int pg_sh = 0;
    LOCKS_REQUIRE(dc_geometry(head_dim, page, &pg_sh),
                  "locks_decode_dense: head_dim %d / page %d outside {64,128,256} x {16,32,64}", head_dim, page);
    LOCKS_REQUIRE(G >= 1 && G <= 16, "locks_decode_dense: G=%d outside [1, 16]", G);
    LOCKS_REQUIRE(split >= 1 && split <= MAX_SPLIT, "locks_decode_dense: split %d outside [1, %d]", split, MAX_SPLIT);
    LOCKS_REQUIRE(num_blocks >= 1 && bt_cols >= 1, "locks_decode_dense: empty geometry");
    LOCKS_REQUIRE(k_stride_tok % 8 == 0 && v_stride_tok % 8 == 0 && k_stride_block % 8 == 0 &&
                  v_stride_block % 8 == 0 && k_stride_head % 8 == 0 && v_stride_head % 8 == 0 &&
                  q_stride_req % 8 == 0 && q_stride_head % 8 == 0,
                  "locks_decode_dense: q/K/V strides must be multiples of 8 elements (16-byte loads)");
    LOCKS_REQUIRE(out_stride_req % 4 == 0 && out_stride_head % 4 == 0,
                  "locks_decode_dense: out strides must be multiples of 4 elements");
    LOCKS_REQUIRE(q && k_cache && v_cache && block_table && seq_lens && m_part && l_part && acc_part && out,
                  "locks_decode_dense: null pointer argument");
    if (n_req == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
#define LAUNCH_D(DV)                                                                                \
    hipLaunchKernelGGL((decode_split_kernel<false, true, DENSE_NST, CPOL_NT, DV>), dim3(split, n_kv, n_req), \
                       dim3(DC_BLK), 0, st, q, (long)q_stride_req, (long)q_stride_head, k_cache,    \
                       (long)k_stride_block, (long)k_stride_tok, (long)k_stride_head, v_cache,      \
                       (long)v_stride_block, (long)v_stride_tok, (long)v_stride_head, num_blocks,   \
                       block_table, (long)bt_stride, bt_cols, nullptr, 0L, 0L, 1, nullptr, 0L,      \
                       seq_lens, m_part, l_part, acc_part, G, split, 1, sm_scale, pg_sh,            \
                       nullptr, nullptr, 0L, 0L, 0, TierSrc{})
    DC_BY_D(head_dim, LAUNCH_D);
#undef LAUNCH_D
    int rc = check_launch("decode_split_kernel<dense>");
    if (rc) return rc;
#define LAUNCH_D(DV)                                                                                \
    hipLaunchKernelGGL(decode_merge_heads_kernel<DV>, dim3(G, n_kv, n_req), dim3(MH_BLK), 0, st,    \
                       m_part, l_part, acc_part, nullptr, 0L, 1, seq_lens, bt_cols, out,            \
                       (long)out_stride_req, (long)out_stride_head, out_is_f32, G, split, split, 1, \
                       page)
    DC_BY_D(head_dim, LAUNCH_D);
#undef LAUNCH_D
    return check_launch("decode_merge_heads_kernel");
}

// Device address of `scratch` per device (the array's host-side name is not
// a device address).  Resolved once per device with that device current.
static std::mutex g_scratch_mu;
static uint8_t* g_scratch_ptr[64];

static int scratch_on_current_device(uint8_t** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    LOCKS_REQUIRE(e == hipSuccess && dev >= 0 && dev < 64,
                  "locks_decode_fused_noalloc: hipGetDevice failed (%s)", hipGetErrorString(e));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        LOCKS_REQUIRE(e == hipSuccess && p, "locks_decode_fused_noalloc: hipGetSymbolAddress(scratch) "
                      "failed on device %d (%s)", dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

extern "C" int32_t locks_decode_fused_noalloc(
    const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
    const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok, int64_t k_stride_head,
    const uint16_t* v_cache, int64_t v_stride_block, int64_t v_stride_tok, int64_t v_stride_head,
    int32_t num_blocks, const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
    const int32_t* page_table, int64_t pt_stride_req, int64_t pt_stride_head, int32_t pt_cols,
    const int32_t* page_cnt, int64_t cnt_stride, const int32_t* seq_lens,
    void* out, int64_t out_stride_req, int64_t out_stride_head, int32_t out_is_f32,
    int32_t n_req, int32_t n_kv, int32_t G, int32_t head_dim, int32_t page,
    int32_t split, int32_t pps_min, int32_t max_cnt, float sm_scale, void* stream)
{
    LOCKS_REQUIRE(n_req >= 0 && n_kv >= 1 && G >= 1 && G <= 16 && split >= 1 && split <= MAX_SPLIT,
                  "locks_decode_fused_noalloc: bad geometry (n_req=%d n_kv=%d G=%d split=%d)",
                  n_req, n_kv, G, split);
    const long rows = (long)n_req * n_kv;
    const long cnt_bytes = rows * LOCKS_DECODE_COUNTER_STRIDE * 4;
    const long ml = rows * split * G;                    // m or l floats
    // every region starts 256-byte aligned: the fused kernel stores and
    // merges the partials with 16-byte vector accesses, and an odd
    // n_req x n_kv x split x G would otherwise leave acc_part 8-byte aligned
    auto up256 = [](long b) { return (b + 255) & ~255L; };
    const long off_m = up256(cnt_bytes), off_l = off_m + up256(ml * 4), off_acc = off_l + up256(ml * 4);
    const long need = off_acc + ml * (long)head_dim * 4;
    LOCKS_REQUIRE(need <= LOCKS_NOALLOC_SCRATCH_BYTES,
                  "locks_decode_fused_noalloc: n_req=%d x n_kv=%d x split=%d x G=%d needs %ld B of "
                  "scratch, more than its %ld B (use locks_decode_fused with caller buffers)",
                  n_req, n_kv, split, G, need, (long)LOCKS_NOALLOC_SCRATCH_BYTES);
    uint8_t* base = nullptr;
    if (int rc = scratch_on_current_device(&base)) return rc;
    if (n_req == 0) return 0;
    int* counters = reinterpret_cast<int*>(base);
    float* m_part = reinterpret_cast<float*>(base + off_m);
    float* l_part = reinterpret_cast<float*>(base + off_l);
    float* acc_part = reinterpret_cast<float*>(base + off_acc);
    // the counters must start at zero: a previous call leaves them zero, but
    // this array is shared by every call on the GPU, so clear them here (a
    // fill kernel, which a HIP graph may capture)
    const int n_ctr = (int)(rows * LOCKS_DECODE_COUNTER_STRIDE);
    hipLaunchKernelGGL(zero_i32_kernel, dim3((unsigned)cdiv(n_ctr, 256)), dim3(256), 0,
                       (hipStream_t)stream, counters, n_ctr);
    if (int rc = check_launch("zero_i32_kernel")) return rc;
    return locks_decode_fused(q, q_stride_req, q_stride_head, k_cache, k_stride_block, k_stride_tok,
                              k_stride_head, v_cache, v_stride_block, v_stride_tok, v_stride_head,
                              num_blocks, block_table, bt_stride, bt_cols, page_table, pt_stride_req,
                              pt_stride_head, pt_cols, page_cnt, cnt_stride, seq_lens, m_part, l_part,
                              acc_part, counters, out, out_stride_req, out_stride_head, out_is_f32,
                              n_req, n_kv, G, head_dim, page, split, pps_min, max_cnt, sm_scale,
                              stream);
}
