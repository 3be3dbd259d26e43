// LOCKS on MLA (one latent KV head shared by all query heads) for gfx950:
// latent page scorer, split-K sparse decode over the selected pages, merge.
//
// Semantics (reference, paths under src/locks/):
//   page score  selection/mla_score_torch.py:27-48 -- max over heads and
//               valid tokens of (q_c . khat_t + q_rope . k_rope_t) * scale;
//               khat is the page summary's reconstruction of the latent.
//   selection   selection/mla_score_torch.py:51-73 (sink + recent window
//               forced inside the budget, top-scored middle) -- served by
//               locks_select_nrm_topb with G = 1, "max" combine.
//   attention   backend/mla_attn.py:178-201 -- softmax over the selected
//               tokens of q . [latent | rope] * scale, o = P . latent, lse.
//
// The page summary is the rki4 record of the latent block (d = kv_lora_rank
// = 512: mean + rank-8 int4 basis + int8 coefficients, built by
// locks_build_rki4) -- the reference keeps fp32 factors Lf, Rf instead
// (mla_select.py:69-108), larger than the page itself; the RoPE keys are
// read exact (bf16) straight from the cache.  Per (page): 2738 B of summary
// + 2048 B of RoPE keys.  With the int8 RoPE summary (rk8: per token 64
// int8 keys, rks: one bf16 scale, absmax / 127 -- 1056 B per page) the
// scorer reads 3794 B per page, and q_rope is int8-quantized per head like
// q_c, so the RoPE term is one i8 matrix-core dot per page.
//
//   tok[h][t] = cs_t sum_c c8[t][c] qt[h][c] + mud[h] + q_rope[h] . k_rope[t]
//   qt[h][c]  = (sum_d V4[c][d] q8[h][d]) qs[h] vs[c]
//   mud[h]    = (sum_d mu8[d] q8[h][d]) qs[h] mus
//   score[p]  = scale * max_{h < H, t} tok[h][t]
//   (int8 RoPE summary: q_rope[h] . k_rope[t] -> (qr8[h] . rk8[t]) qrs[h] rks[t])
#include "locks_common.h"
#include "locks_hip.h"

namespace locks {

constexpr int ML_D = 512;                    // kv_lora_rank
constexpr int ML_DR = 64;                    // RoPE dims
constexpr int ML_HS = ML_D + ML_DR;          // cache row (576)
constexpr int ML_PG = 16;
constexpr int ML_RNK = 8;
constexpr int ML_H = 16;                     // query heads (upper bound)
constexpr int ML_WAVES = 4;
constexpr int ML_BLK = ML_WAVES * kWave;
constexpr int ML_VROW = ML_RNK * ML_D / 2;   // 2048 B packed V per page
constexpr int ML_MAX_CHUNK = 1024;
// Per-wave LDS stage of one unit (2 pages), filled by LDS DMA
// (global_load_lds_dwordx4: lane L of an instruction writes the 16 bytes at
// 16 L of the instruction's 1-KB window, from its own source address).
// Rows are stored unpadded with their 64-byte blocks permuted by an XOR of
// the row index, so the MFMA-order reads (16 rows at once, the same part of
// each) spread over four bank groups; the DMA fetches, for each LDS slot,
// the part that belongs there.  (Permuting the 16-byte parts themselves
// would spread the reads over all banks but break each lane quad's 64
// contiguous source bytes into four requests: measured 15.6 vs 14.2 us.)
constexpr int ML_CPOL_NT = 2;
typedef __attribute__((address_space(3))) void* ml_lds_ptr;                // buffer-load cache policy: non-temporal
constexpr int MS_V = 0;                      // 16 (page, column) rows x 256 B packed V
constexpr int MS_MU = 4096;                  // 2 x 512 centroid
constexpr int MS_RP = 5120;                  // 32 (page, token) RoPE rows
// RoPE rows: exact bf16 keys (128 B) or int8 keys (64 B); then the small
// rows (c8 | cs | vs | RQ: the int8 keys' bf16 scales) and the centroid terms
template <bool RQ>
struct MsGeom {
    static constexpr int RROWB = RQ ? 64 : 128;
    static constexpr int NRI = RQ ? 2 : 4;               // DMA instructions of the RoPE rows
    static constexpr int SM = MS_RP + 32 * RROWB;        // small rows
    static constexpr int S_C8 = SM, S_CS = SM + 256, S_VS = SM + 320, S_RS = SM + 352;
    static constexpr int NSM = RQ ? 26 : 22;             // 16-byte chunks of the small rows
    static constexpr int MD = SM + 16 * NSM;             // 2 x 16 fp32 centroid terms
    static constexpr int BYTES = MD + 128;
};
// LDS slot (16-byte part index) of part p of a stage row R, and its
// inverse: packed V (256-B rows, four blocks), exact RoPE (128-B rows, two
// blocks; two rows per 256-B bank span), int8 RoPE (64-B rows, one block)
__device__ __forceinline__ int ms_vslot(int R, int p) { return (((p >> 2) ^ (R & 3)) << 2) | (p & 3); }
__device__ __forceinline__ int ms_rslot(int R, int p) { return (((p >> 2) ^ ((R >> 1) & 1)) << 2) | (p & 3); }
__device__ __forceinline__ int ms_vpos(int R, int p) { return MS_V + R * 256 + (ms_vslot(R, p) << 4); }
template <bool RQ>
__device__ __forceinline__ int ms_rpos(int R, int p) {
    return RQ ? MS_RP + R * 64 + (p << 4) : MS_RP + R * 128 + (ms_rslot(R, p) << 4);
}
constexpr int ML_RK_BLOCK = ML_PG * ML_DR;   // int8 RoPE keys per block (1024 B)

__device__ __forceinline__ v4i perm_even_odd(const uint4 n) {
    // 16 int8 in d order -> even d of the window first, then odd d (the
    // order the int4 nibble operand of the projection uses)
    return v4i{(int)__builtin_amdgcn_perm(n.y, n.x, 0x06040200u), (int)__builtin_amdgcn_perm(n.w, n.z, 0x06040200u),
               (int)__builtin_amdgcn_perm(n.y, n.x, 0x07050301u), (int)__builtin_amdgcn_perm(n.w, n.z, 0x07050301u)};
}

// 16-byte non-temporal load (global_load_dwordx4 ... nt)
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const v4u x = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(x.x, x.y, x.z, x.w);
}

// ---------------------------------------------------------------------------
// latent page scorer: grid (chunks, requests), 4 waves; unit = 2 pages
// ---------------------------------------------------------------------------
// RQ: RoPE term from the int8 RoPE summary (rk8, rks) with int8 q_rope;
// else from the exact bf16 keys of the cache with bf16 q_rope.
template <bool RQ>
__global__ __launch_bounds__(ML_BLK) void mla_score_kernel(
    const uint16_t* __restrict__ q, long q_sr, long q_sh,
    const uint8_t* __restrict__ v4, const uint16_t* __restrict__ vs,
    const int8_t* __restrict__ c8, const uint16_t* __restrict__ cs,
    const int8_t* __restrict__ mu8, const uint16_t* __restrict__ mus,
    const int8_t* __restrict__ rk8, const uint16_t* __restrict__ rks,
    const uint16_t* __restrict__ cache, long c_sb, long c_st,
    int NB, const int* __restrict__ bt, long bt_sr, int bt_cols,
    const int* __restrict__ nsh, float* __restrict__ score, long sc_sr, int MP,
    int H, float scale, int chunk)
{
    using GM = MsGeom<RQ>;
    const int z = blockIdx.x, r = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int P = min(nsh[r], MP);
    const int c0 = z * chunk;
    const int c1 = min(c0 + chunk, P);
    if (c0 >= c1) return;

    // two stages per wave as separate LDS objects (a unit's reads never share
    // an object with the next unit's DMA); the int8 q rows and the q_rope rows
    // live in the second stages until the q operands are built
    __shared__ __attribute__((aligned(16))) uint8_t sa_l[ML_WAVES][GM::BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t sb_l[ML_WAVES][GM::BYTES];
    __shared__ float qss[ML_H];
    __shared__ float qrss[ML_H];                                        // RQ: q_rope scale per head
    extern __shared__ __attribute__((aligned(16))) int bt_l[];          // block ids of the chunk
    static_assert((ML_H + 1) * ML_D + ML_H * ML_DR * 2 <= ML_WAVES * GM::BYTES, "q rows fit the second stages");
    int8_t (*q8s)[ML_D] = reinterpret_cast<int8_t (*)[ML_D]>(&sb_l[0][0]);                   // row 16 = zeros
    uint16_t (*qrs)[ML_DR] = reinterpret_cast<uint16_t (*)[ML_DR]>(&sb_l[0][0] + (ML_H + 1) * ML_D);  // RQ: int8 in the first half

    // ---- prologue: q rows of this wave's heads and the block ids in one
    // round trip; the first unit's DMA is issued before q is quantized
    // (absmax / 127 per head), so the quantization overlaps it
    // Unconditional loads (heads past H re-read head H - 1 and are zeroed
    // or never stored): a guarded load is waited for at its branch join,
    // which would serialise the heads' round trips.
    constexpr int QH = ML_H / ML_WAVES;
    uint4 qw[QH], qrw[QH];
#pragma unroll
    for (int i = 0; i < QH; ++i) {
        const int h = min(wave + ML_WAVES * i, H - 1);
        const uint16_t* qh = q + (long)r * q_sr + (long)h * q_sh;
        qw[i] = *reinterpret_cast<const uint4*>(qh + 8 * lane);
        qrw[i] = make_uint4(0u, 0u, 0u, 0u);
        if constexpr (!RQ) qrw[i] = *reinterpret_cast<const uint4*>(qh + ML_D + 8 * (lane & 7));
    }
    // RQ: the wave's QH q_rope rows side by side, lane l < 8 QH holding dims
    // 8 (l & 7) .. of head wave + QH (l >> 3)
    const int hr = wave + ML_WAVES * (lane >> 3);
    const bool hr_ok = RQ && lane < 8 * QH && hr < H;
    uint4 qrw8 = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (RQ)
        qrw8 = *reinterpret_cast<const uint4*>(q + (long)r * q_sr + (long)min(hr, H - 1) * q_sh + ML_D + 8 * (lane & 7));
    for (int i = tid; i < c1 - c0; i += ML_BLK) {
        const int b = bt[(long)r * bt_sr + min(c0 + i, bt_cols - 1)];
        bt_l[i] = min(max(b, 0), NB - 1);
    }
    __syncthreads();
    const int r16 = lane & 15, kg = lane >> 4;
    const int n_units = cdiv(c1 - c0, 2);

    // ---- the unit DMA: per lane and instruction a source address; the LDS
    // slot of lane L is fixed (16 L into the instruction's 1-KB window)
    // small rows: lane -> (field base, page, byte offset) once for all units
    const uint8_t* sm_base;
    int sm_stride, sm_page, sm_off;
    if (lane < 16) { sm_base = reinterpret_cast<const uint8_t*>(c8); sm_stride = ML_PG * ML_RNK; sm_page = lane >> 3; sm_off = (lane & 7) * 16; }
    else if (lane < 20) { sm_base = reinterpret_cast<const uint8_t*>(cs); sm_stride = ML_PG * 2; sm_page = (lane - 16) >> 1; sm_off = ((lane - 16) & 1) * 16; }
    else if (lane < 22 || !RQ) { sm_base = reinterpret_cast<const uint8_t*>(vs); sm_stride = ML_RNK * 2; sm_page = (lane - 20) & 1; sm_off = 0; }
    else { sm_base = reinterpret_cast<const uint8_t*>(rks); sm_stride = ML_PG * 2; sm_page = ((lane - 22) >> 1) & 1; sm_off = ((lane - 22) & 1) * 16; }
    struct UnitSrc {
        const uint8_t* a[4 + 1 + GM::NRI + 1];      // V x 4, centroid, RoPE rows, small rows
    };
    constexpr int NI = 4 + 1 + GM::NRI + 1;
    auto unit_src = [&](int u, uint32_t& mus_off) -> UnitSrc {
        const int p0 = 2 * u, last = c1 - c0 - 1;
        const long b0 = bt_l[min(p0, last)], b1 = bt_l[min(p0 + 1, last)];   // tail pair repeats the last page
        UnitSrc f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {               // V rows 4 i .. 4 i + 3 (page i >> 1)
            const int R = 4 * i + (lane >> 4), pq = ms_vslot(R, lane & 15);   // the permutation is an involution
            f.a[i] = v4 + ((i >> 1) ? b1 : b0) * ML_VROW + (R & 7) * 256 + pq * 16;
        }
        f.a[4] = reinterpret_cast<const uint8_t*>(mu8) + ((lane >> 5) ? b1 : b0) * ML_D + (lane & 31) * 16;
#pragma unroll
        for (int j = 0; j < GM::NRI; ++j) {
            if constexpr (RQ) {                     // int8 key rows 16 j .. (page j), 4 parts of 16 B
                const int R = 16 * j + (lane >> 2), pq = lane & 3;
                f.a[5 + j] = reinterpret_cast<const uint8_t*>(rk8) + (j ? b1 : b0) * ML_RK_BLOCK + (R & 15) * ML_DR + pq * 16;
            } else {                                // exact key rows 8 j .. (page j >> 1), 8 parts of 16 B
                const int R = 8 * j + (lane >> 3), pq = ms_rslot(R, lane & 7);
                f.a[5 + j] = reinterpret_cast<const uint8_t*>(cache + ((j >> 1) ? b1 : b0) * c_sb + (long)(R & 15) * c_st + ML_D + 8 * pq);
            }
        }
        f.a[NI - 1] = sm_base + (sm_page ? b1 : b0) * sm_stride + sm_off;
        mus_off = (uint32_t)((lane & 1) ? b1 : b0);
        return f;
    };
    uint32_t fmus = 0u;                               // centroid scale of page lane & 1
    auto issue = [&](const UnitSrc& f, uint32_t mus_blk, uint8_t* st) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint8_t* src = f.a[i];
            __builtin_amdgcn_global_load_lds(src, (ml_lds_ptr)(st + MS_V + 1024 * i), 16, 0, ML_CPOL_NT);
        }
        {
            const uint8_t* src = f.a[4];
            __builtin_amdgcn_global_load_lds(src, (ml_lds_ptr)(st + MS_MU), 16, 0, ML_CPOL_NT);
        }
#pragma unroll
        for (int j = 0; j < GM::NRI; ++j) {
            const uint8_t* src = f.a[5 + j];
            __builtin_amdgcn_global_load_lds(src, (ml_lds_ptr)(st + MS_RP + 1024 * j), 16, 0, ML_CPOL_NT);
        }
        // the scale rows share cache lines with neighbouring blocks: default policy
        if (lane < GM::NSM) {
            const uint8_t* src = f.a[NI - 1];
            __builtin_amdgcn_global_load_lds(src, (ml_lds_ptr)(st + GM::SM), 16, 0, 0);
        }
        fmus = (uint32_t)mus[mus_blk];
    };
    auto pin = [&](const UnitSrc& f) {              // DMA sources stay allocated until the unit ends
#pragma unroll
        for (int i = 0; i < NI; ++i) asm volatile("" :: "v"(f.a[i]));
    };
    // q rows resident before the first unit's DMA queues behind them (the
    // compiler could not tell they are, and would wait for the DMA too)
    __builtin_amdgcn_s_waitcnt(0x0070);
    if (wave < n_units) {
        uint32_t mb;
        const UnitSrc f0 = unit_src(wave, mb);
        pin(f0);
        issue(f0, mb, sa_l[wave]);
    }

    // int8 round trip of one head's row, 8 values per lane: qs = max(absmax,
    // 1e-8) / 127 over the wave, v = rint(a / qs) with the correctly rounded
    // quotient: a * (1 / qs) is within 2 ulp of it and decides the rounding
    // unless it lies within 2^-15 of a half-integer; those (rare) lanes redo
    // the division.  Returns qs; packs the 8 values (zeros when !valid).
    // g8: the row is 8 lanes wide (absmax over each 8-lane group) instead
    // of the whole wave
    auto quant8 = [&](const uint4 w, bool valid, uint32_t (&pk)[2], bool g8) -> float {
        float a[8];
        {
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) { a[2 * e] = bf16lo(ws[e]); a[2 * e + 1] = bf16hi(ws[e]); }
        }
        float am = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(a[e]));
        if (g8) {
            // quad swaps, then the half-row mirror (lane j <-> 7 - j of 8)
            am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0xB1, 0xF, 0xF, false)));
            am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0x4E, 0xF, 0xF, false)));
            am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0x141, 0xF, 0xF, false)));
        } else {
            am = wave_max(am);
        }
        const float qs = fmaxf(am, 1e-8f) / 127.f;
        const float inv = 1.f / qs;
        int iv[8];
        bool near = false;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float y = a[e] * inv;
            const float ry = rintf(y);
            near |= fabsf(fabsf(y - ry) - 0.5f) < 0x1p-15f;
            iv[e] = (int)ry;
        }
        if (__builtin_expect(__ballot(near) != 0ull, 0)) {
            if (near) {
#pragma unroll
                for (int e = 0; e < 8; ++e) iv[e] = (int)rintf(__fdiv_rn(a[e], qs));
            }
        }
        pk[0] = pk[1] = 0u;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int v = valid ? iv[e] : 0;
            pk[e >> 2] |= ((uint32_t)(uint8_t)v) << (8 * (e & 3));
        }
        return qs;
    };
    for (int i = tid; i < ML_D / 4; i += ML_BLK) reinterpret_cast<int*>(&q8s[ML_H][0])[i] = 0;
#pragma unroll
    for (int i = 0; i < QH; ++i) {
        const int h = wave + ML_WAVES * i;
        uint32_t pk[2];
        const float qs = quant8(qw[i], h < H, pk, false);
        *reinterpret_cast<uint2*>(&q8s[h][8 * lane]) = make_uint2(pk[0], pk[1]);
        if constexpr (!RQ) {
            if (lane < ML_DR / 8) *reinterpret_cast<uint4*>(&qrs[h][8 * lane]) = (h < H) ? qrw[i] : make_uint4(0u, 0u, 0u, 0u);
        }
        if (lane == 0) qss[h] = (h < H) ? qs : 0.f;
    }
    if constexpr (RQ) {
        // q_rope: the same round trip over each head's 64 dims, the wave's
        // QH heads at once
        uint32_t pr[2];
        const float qsr = quant8(qrw8, hr_ok, pr, true);
        if (lane < 8 * QH) {
            *reinterpret_cast<uint2*>(reinterpret_cast<int8_t*>(&qrs[hr][0]) + 8 * (lane & 7)) = make_uint2(pr[0], pr[1]);
            if ((lane & 7) == 0) qrss[hr] = hr_ok ? qsr : 0.f;
        }
    }
    // barrier on the q rows while the first unit's DMA is in flight: the
    // compiler's LDS fences would also wait for the DMA (it writes LDS), so
    // the LDS completion wait and the barrier are explicit, the asm a
    // compiler memory barrier
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const uint32_t MH = 0xF0F0F0F0u;
    // q operands shared by every unit: projection B (column j = head j),
    // RoPE B (column = head), per-head scale of this lane's column
    v4i Bq[4][2];
    {
        const int hrow = r16 < H ? r16 : ML_H;
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
            Bq[k4][0] = perm_even_odd(*reinterpret_cast<const uint4*>(&q8s[hrow][128 * k4 + 32 * kg]));
            Bq[k4][1] = perm_even_odd(*reinterpret_cast<const uint4*>(&q8s[hrow][128 * k4 + 32 * kg + 16]));
        }
    }
    // RoPE B operand: exact form, bf16 q_rope of head r16 (k-step s, slot
    // kg: dims 32 s + 8 kg ..); int8 form, lane group kg holds dims
    // 16 kg .. 16 kg + 15 of head r16 (the same dims as the A rows' bytes)
    v8bf Br[2];
    v4i Br8 = {0, 0, 0, 0};
    float qrsj = 0.f;
    if constexpr (RQ) {
        const uint4 w = *reinterpret_cast<const uint4*>(reinterpret_cast<const int8_t*>(&qrs[r16][0]) + 16 * kg);
        Br8 = v4i{(int)w.x, (int)w.y, (int)w.z, (int)w.w};
        qrsj = qrss[r16];
    } else {
#pragma unroll
        for (int s = 0; s < 2; ++s)
            Br[s] = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(&qrs[r16][32 * s + 8 * kg]));
    }
    const float qsj = qss[r16];
    const bool col_ok = r16 < H;
    // q rows consumed: the second stages are free (explicit for the same reason)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // a unit's page scores are stored after the next unit's wait (vmcnt(0)
    // would otherwise also wait for the stores just issued)
    float pend_m[2] = {0.f, 0.f};
    long pend_at = -1;
    int pend_n = 0;
    auto flush = [&]() {
        if (lane == 0 && pend_at >= 0) {
            score[pend_at] = pend_m[0];
            if (pend_n > 1) score[pend_at + 1] = pend_m[1];
        }
    };
    auto score_unit = [&](int u, uint8_t* st, uint8_t* st_next) {
        __builtin_amdgcn_s_waitcnt(0x0070);          // this unit's rows have landed in the stage
        wave_lds_sync();
        flush();
        // centroid scales of the pair, before the next unit's load replaces them
        const uint32_t mus0 = (uint32_t)__builtin_amdgcn_readlane((int)fmus, 0);
        const uint32_t mus1 = (uint32_t)__builtin_amdgcn_readlane((int)fmus, 1);
        const bool more = u + ML_WAVES < n_units;
        UnitSrc nf;
        uint32_t nmb = 0u;
        if (more) nf = unit_src(u + ML_WAVES, nmb);
        const int p0 = c0 + 2 * u;
        const int nvalid = min(2, c1 - p0);

        // ---- projection (A = the 16 V rows of the pair, row 4a + b <->
        // page b & 1, column 2a + (b >> 1); B = int8 q) and the centroid
        // term (A rows 0/1 = the two mu rows, same B); every read of this
        // stage's V and centroid is issued before the next unit's DMA
        const int i_pg = r16 & 1, i_c = 2 * (r16 >> 2) + ((r16 >> 1) & 1);
        const int Rv = i_pg * 8 + i_c;
        uint4 wv[4], wm[4][2];
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
            wv[k4] = *reinterpret_cast<const uint4*>(st + ms_vpos(Rv, k4 * 4 + kg));
            wm[k4][0] = wm[k4][1] = make_uint4(0u, 0u, 0u, 0u);
            if (r16 < 2) {
                wm[k4][0] = *reinterpret_cast<const uint4*>(st + MS_MU + r16 * ML_D + 128 * k4 + 32 * kg);
                wm[k4][1] = *reinterpret_cast<const uint4*>(st + MS_MU + r16 * ML_D + 128 * k4 + 32 * kg + 16);
            }
        }
        const uint32_t vsw0 = *reinterpret_cast<const uint32_t*>(st + GM::S_VS + 0 * 16 + kg * 4);
        const uint32_t vsw1 = *reinterpret_cast<const uint32_t*>(st + GM::S_VS + 1 * 16 + kg * 4);
        if (more) issue(nf, nmb, st_next);
        v4i acc = {0, 0, 0, 0}, accm = {0, 0, 0, 0};
#pragma unroll
        for (int k4 = 0; k4 < 4; ++k4) {
            const uint4 w = wv[k4];
            const v4i a0 = {(int)((w.x << 4) & MH), (int)((w.y << 4) & MH), (int)(w.x & MH), (int)(w.y & MH)};
            const v4i a1 = {(int)((w.z << 4) & MH), (int)((w.w << 4) & MH), (int)(w.z & MH), (int)(w.w & MH)};
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, Bq[k4][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, Bq[k4][1], acc, 0, 0, 0);
            accm = __builtin_amdgcn_mfma_i32_16x16x64_i8(perm_even_odd(wm[k4][0]), Bq[k4][0], accm, 0, 0, 0);
            accm = __builtin_amdgcn_mfma_i32_16x16x64_i8(perm_even_odd(wm[k4][1]), Bq[k4][1], accm, 0, 0, 0);
        }
        // qt[v] = qt[head r16][page v & 1][column 2kg + (v >> 1)]; the 1/16 of
        // the high-nibble operand rides on the power-of-two column scale
        float qt[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t w = (v & 1) ? vsw1 : vsw0;
            const float vsc = ((v >> 1) ? bf16hi(w) : bf16lo(w)) * 0.0625f;
            qt[v] = (float)acc[v] * qsj * vsc;
        }
        // centroid term of (page v, head r16) lives in lanes kg = 0, v = 0/1
        float* md = reinterpret_cast<float*>(st + GM::MD);
        if (kg == 0) {
#pragma unroll
            for (int v = 0; v < 2; ++v)
                md[v * 16 + r16] = (float)accm[v] * qsj * bf16lo(v ? mus1 : mus0);
        }
        wave_lds_sync();

        // ---- per page: token reconstruction + RoPE, max over (t, h) -------
#pragma unroll
        for (int pg = 0; pg < 2; ++pg) {
            v4f tk = {0.f, 0.f, 0.f, 0.f};
            const uint32_t cw = *reinterpret_cast<const uint16_t*>(st + GM::S_C8 + pg * 128 + r16 * 8 + 2 * kg);
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const float a = (float)(int8_t)(cw >> (8 * hh));
                tk = __builtin_amdgcn_mfma_f32_16x16x4f32(a, qt[2 * hh + pg], tk, 0, 0, 0);
            }
            v4f rp = {0.f, 0.f, 0.f, 0.f};
            const int Rr = pg * 16 + r16;               // RoPE row of this lane's token
            if constexpr (RQ) {
                // rows = the page's 16 tokens, 16 int8 dims per lane group
                const uint4 w = *reinterpret_cast<const uint4*>(st + ms_rpos<RQ>(Rr, kg));
                const v4i ri = __builtin_amdgcn_mfma_i32_16x16x64_i8(v4i{(int)w.x, (int)w.y, (int)w.z, (int)w.w},
                                                                     Br8, v4i{0, 0, 0, 0}, 0, 0, 0);
                const uint2 rsw = *reinterpret_cast<const uint2*>(st + GM::S_RS + pg * 32 + kg * 8);
                rp[0] = (float)ri[0] * qrsj * bf16lo(rsw.x);
                rp[1] = (float)ri[1] * qrsj * bf16hi(rsw.x);
                rp[2] = (float)ri[2] * qrsj * bf16lo(rsw.y);
                rp[3] = (float)ri[3] * qrsj * bf16hi(rsw.y);
            } else {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const v8bf a = __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4*>(st + ms_rpos<RQ>(Rr, 4 * s + kg)));
                    rp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, Br[s], rp, 0, 0, 0);
                }
            }
            const uint2 csw = *reinterpret_cast<const uint2*>(st + GM::S_CS + pg * 32 + kg * 8);
            const float mud = md[pg * 16 + r16];
            const float t0 = fmaf(tk[0], bf16lo(csw.x), rp[0]);
            const float t1 = fmaf(tk[1], bf16hi(csw.x), rp[1]);
            const float t2 = fmaf(tk[2], bf16lo(csw.y), rp[2]);
            const float t3 = fmaf(tk[3], bf16hi(csw.y), rp[3]);
            float m = col_ok ? fmaxf(fmaxf(t0, t1), fmaxf(t2, t3)) + mud : -INFINITY;
            m = wave_max(m);
            pend_m[pg] = m * scale;
        }
        pend_at = (long)r * sc_sr + p0;
        pend_n = nvalid;
        if (more) pin(nf);
        wave_lds_sync();                                 // stage reused by the unit after next
    };
    for (int u = wave; u < n_units; u += 2 * ML_WAVES) {
        score_unit(u, sa_l[wave], sb_l[wave]);
        if (u + ML_WAVES < n_units) score_unit(u + ML_WAVES, sb_l[wave], sa_l[wave]);
    }
    flush();
}

// ---------------------------------------------------------------------------
// int8 RoPE summary of listed blocks: one wave per block, lane = (token
// lane >> 2, 16 dims 16 (lane & 3) ..); per token scale = max(absmax / 127,
// 1e-8) (the rki4 token-scale rule) rounded to bf16, key = clamp(rint(k /
// bf16 scale), +-127); the bf16 scale is stored
// ---------------------------------------------------------------------------
constexpr int MR_WAVES = 4;
__global__ __launch_bounds__(MR_WAVES * kWave) void mla_rope_quant_kernel(
    const uint16_t* __restrict__ cache, long c_sb, long c_st, int NB,
    const int* __restrict__ blocks, int n, const int* __restrict__ n_dev, int8_t* __restrict__ rk8,
    uint16_t* __restrict__ rks)
{
    const int i = blockIdx.x * MR_WAVES + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (n_dev) n = min(n, *n_dev);                                 // device-side count
    if (i >= n) return;
    const int b = blocks[i];
    if (b < 0 || b >= NB) return;                                  // skipped id
    const int t = lane >> 2, part = lane & 3;
    const uint16_t* src = cache + (long)b * c_sb + (long)t * c_st + ML_D + 16 * part;
    const uint4 w0 = *reinterpret_cast<const uint4*>(src);
    const uint4 w1 = *reinterpret_cast<const uint4*>(src + 8);
    const uint32_t ws[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    float x[16];
#pragma unroll
    for (int e = 0; e < 8; ++e) { x[2 * e] = bf16lo(ws[e]); x[2 * e + 1] = bf16hi(ws[e]); }
    float am = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) am = fmaxf(am, fabsf(x[e]));
    am = fmaxf(am, __shfl_xor(am, 1));
    am = fmaxf(am, __shfl_xor(am, 2));
    // the stored bf16 scale is the one the keys are quantized with, so the
    // scorer's dequantization k8 * scale uses exactly the quantization step
    const uint16_t sb = f32_to_bf16(fmaxf(__fdiv_rn(am, 127.f), 1e-8f));
    const float sc = __uint_as_float((uint32_t)sb << 16);
    uint32_t pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int v = (int)fminf(fmaxf(rintf(__fdiv_rn(x[e], sc)), -127.f), 127.f);
        pk[e >> 2] |= ((uint32_t)(uint8_t)v) << (8 * (e & 3));
    }
    *reinterpret_cast<uint4*>(rk8 + (long)b * ML_RK_BLOCK + t * ML_DR + 16 * part) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    if (part == 0) rks[(long)b * ML_PG + t] = sb;
}

// ---------------------------------------------------------------------------
// split-K sparse decode over the selected latent pages
// ---------------------------------------------------------------------------
// Workgroup = 4 waves = one split of one request.  A page (16 tokens x 576
// bf16 = 18 KB) is DMA'd with global_load_lds_dwordx4 into one of two
// workgroup stages while the other is consumed.  S = K Q^T is split over the
// waves by head-dim k-steps (partials summed through LDS in a fixed order,
// so every wave holds the identical S); each wave then owns a 128-d slice of
// the 512-d output for O^T += V^T P^T.  All stage and partial accesses are
// inline-asm LDS ops: the compiler cannot tell them from the DMA in flight
// and would otherwise wait for it before every access.
constexpr int MD_ROWB = ML_HS * 2 + 16;               // padded token row (1168 B)
constexpr int MD_PAGE_B = ML_PG * MD_ROWB;            // 18688 B per stage
constexpr int MD_IDS = 256;                           // page ids staged per batch
constexpr int MD_MAX_SPLIT = 512;
constexpr int CPOL_NT_MLA = 2;                        // non-temporal DMA (dense: every page read once)
typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)(p);
}
__device__ __forceinline__ v4i ds_read16(uint32_t a) {
    v4i v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a));
    return v;
}
__device__ __forceinline__ void ds_write16(uint32_t a, v4i x) {
    asm volatile("ds_write_b128 %0, %1" : : "v"(a), "v"(x));
}
// Wait for the outstanding LDS ops; the loaded registers pass through the
// wait as operands so no use of them can be scheduled before it.
__device__ __forceinline__ void lgkm_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void lgkm_wait(v4i& a, v4i& b, v4i& c, v4i& d) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) :: "memory");
}
__device__ __forceinline__ void lgkm_wait(v4i& a, v4i& b, v4i& c, v4i& d, v4i& e) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e) :: "memory");
}

// DENSE: every page of the row in logical order (page count from seq_len, no
// page table) -- the dense full-cache comparator.  NST: page stages per
// workgroup (NST - 1 pages in flight while one is consumed).  KVPOL: cache
// policy bits of the page DMA.
constexpr int vm_wait_imm(int n) {                       // s_waitcnt vmcnt(n) lgkmcnt(0)
    return 0x0070 | (n & 15) | ((n >> 4) << 14);
}
template <bool DENSE = false, int NST = 2, int KVPOL = 0>
__global__ __launch_bounds__(ML_BLK) void mla_decode_split_kernel(
    const uint16_t* __restrict__ q, long q_sr, long q_sh,
    const uint16_t* __restrict__ cache, long c_sb, long c_st, int NB,
    const int* __restrict__ bt, long bt_sr, int bt_cols,
    const int* __restrict__ ptab, long pt_sr, int pt_cols, const int* __restrict__ pcnt,
    const int* __restrict__ seq_lens, float* __restrict__ m_part, float* __restrict__ l_part,
    float* __restrict__ acc_part, int H, int split, int pps_min, float scale)
{
    static_assert(NST >= 2 && NST <= 4, "page stages");
    const int sp = blockIdx.x, r = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, kg = lane >> 4;
    // The page count, this thread's first page id assuming pps == pps_min
    // (the usual sparse case) and the q rows are loaded together, so the
    // page ids do not wait for the count.
    const int js = sp * pps_min + tid;
    const int pt_spec = DENSE ? 0 : ptab[(long)r * pt_sr + min(js, pt_cols - 1)];

    __shared__ __attribute__((aligned(16))) uint8_t stg[NST][MD_PAGE_B];
    __shared__ __attribute__((aligned(16))) float spart[ML_WAVES][kWave * 4];
    __shared__ int ids_pt[MD_IDS], ids_blk[MD_IDS];

    // QK k-steps of this wave: 18 steps of 32 dims split 5/5/4/4
    const int s_lo = wave < 2 ? 5 * wave : 10 + 4 * (wave - 2);
    const int s_n = wave < 2 ? 5 : 4;
    v8bf qb[5];
    {
        const uint16_t* qp = q + (long)r * q_sr + (long)r16 * q_sh + 8 * kg;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            uint4 w = make_uint4(0u, 0u, 0u, 0u);
            if (i < s_n && r16 < H) w = *reinterpret_cast<const uint4*>(qp + 32 * (s_lo + i));
            qb[i] = __builtin_bit_cast(v8bf, w);
        }
    }
    const int cnt = DENSE ? min(cdiv(seq_lens[r], ML_PG), bt_cols) : min(pcnt[r], pt_cols);
    const int pps = max(cdiv(cnt, split), pps_min);
    const int j0 = sp * pps;
    if (j0 >= cnt) return;                               // inactive split: no store
    const int j1 = min(j0 + pps, cnt);
    const int seq_len = seq_lens[r];
    float m = -INFINITY, lsum = 0.f;
    v4f o[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) o[b] = v4f{0.f, 0.f, 0.f, 0.f};

    const uint32_t st0 = lds_addr(&stg[0][0]);
    const uint32_t sp_base = lds_addr(&spart[0][0]);
    // DMA of one page: wave w fills token rows 4w .. 4w+3, each row as one
    // 64-chunk and one 8-chunk instruction (rows are padded in LDS, so an
    // instruction never crosses a row)
    auto issue = [&](int slot, int blk) {
        const uint16_t* base = cache + (long)blk * c_sb;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const int t = 4 * wave + q4;
            const uint16_t* row = base + (long)t * c_st;
            __builtin_amdgcn_global_load_lds(row + 8 * lane, (lds_ptr_t)(&stg[slot][t * MD_ROWB]), 16, 0, KVPOL);
            if (lane < 8)
                __builtin_amdgcn_global_load_lds(row + 8 * (64 + lane), (lds_ptr_t)(&stg[slot][t * MD_ROWB + 1024]),
                                                 16, 0, KVPOL);
        }
    };

    for (int jb = j0; jb < j1; jb += MD_IDS) {
        const int nb = min(MD_IDS, j1 - jb);
        __syncthreads();                                      // previous batch fully consumed
        const bool spec = pps == pps_min && jb == j0;         // jb + tid == js
        for (int i = tid; i < nb; i += ML_BLK) {
            const int pt = DENSE ? jb + i : (spec && i == tid) ? pt_spec : ptab[(long)r * pt_sr + jb + i];
            const int ptc = min(max(pt, 0), bt_cols - 1);
            ids_pt[i] = pt;
            ids_blk[i] = min(max(bt[(long)r * bt_sr + ptc], 0), NB - 1);
        }
        __syncthreads();
        // ring of NST stages: page i + NST - 1 is issued (into the slot of
        // page i - 1) once every wave is past page i - 1
#pragma unroll
        for (int k = 0; k < NST - 1; ++k)
            if (k < nb) issue(k, ids_blk[k]);
        for (int i = 0; i < nb; ++i) {
            const int slot = i % NST;
            // this wave's part of page i landed: 8 DMA instructions per page
            // per wave, min(NST - 2, nb - 1 - i) pages issued after it
            const int ahead = min(NST - 2, nb - 1 - i);
            if (ahead <= 0) __builtin_amdgcn_s_waitcnt(vm_wait_imm(0));
            else if (NST > 2 && ahead == 1) __builtin_amdgcn_s_waitcnt(vm_wait_imm(8));
            else if (NST > 3) __builtin_amdgcn_s_waitcnt(vm_wait_imm(16));
            __builtin_amdgcn_s_barrier();                     // every part landed; page i-1 consumed
            if (i + NST - 1 < nb) issue((i + NST - 1) % NST, ids_blk[i + NST - 1]);
            const int pt = ids_pt[i];
            const uint32_t sb = st0 + slot * MD_PAGE_B;
            // ---- partial S^T[t][h] over this wave's k-steps ----------------
            v4f sacc = {0.f, 0.f, 0.f, 0.f};
            v4i ka[5];
#pragma unroll
            for (int k = 0; k < 5; ++k)
                if (k < s_n) ka[k] = ds_read16(sb + r16 * MD_ROWB + (32 * (s_lo + k) + 8 * kg) * 2);
            lgkm_wait(ka[0], ka[1], ka[2], ka[3], ka[4]);
#pragma unroll
            for (int k = 0; k < 5; ++k)
                if (k < s_n)
                    sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, ka[k]), qb[k], sacc, 0, 0, 0);
            ds_write16(sp_base + (wave * kWave + lane) * 16, __builtin_bit_cast(v4i, sacc));
            lgkm_wait();
            __builtin_amdgcn_s_barrier();
            v4i px[4];
#pragma unroll
            for (int w = 0; w < ML_WAVES; ++w) px[w] = ds_read16(sp_base + (w * kWave + lane) * 16);
            lgkm_wait(px[0], px[1], px[2], px[3]);
            v4f sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < ML_WAVES; ++w) sv = sv + __builtin_bit_cast(v4f, px[w]);   // fixed order
            // ---- online softmax (head = lane column) ----------------------
            float s4[4];
            const int pos0 = pt * ML_PG + 4 * kg;
#pragma unroll
            for (int v = 0; v < 4; ++v) s4[v] = (pos0 + v < seq_len && r16 < H) ? sv[v] * scale : -INFINITY;
            float mx = fmaxf(fmaxf(s4[0], s4[1]), fmaxf(s4[2], s4[3]));
            mx = xor32_max(xor16_max(mx));
            const float m_new = fmaxf(m, mx);
            const float m_ref = (m_new == -INFINITY) ? 0.f : m_new;
            const float alpha = __expf(m - m_ref);
            float p[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) p[v] = __expf(s4[v] - m_ref);
            lsum = lsum * alpha + (p[0] + p[1] + p[2] + p[3]);
            m = m_new;
            const v4h pb = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
            // ---- O^T[d][h] += V^T P^T over this wave's 128 dims ------------
            v4i vi[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                vi[j] = ds_read16(sb + (4 * kg + j) * MD_ROWB + (128 * wave + 8 * r16) * 2);
            lgkm_wait(vi[0], vi[1], vi[2], vi[3]);
            uint4 vr[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) vr[j] = __builtin_bit_cast(uint4, vi[j]);
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                v4h a;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t x = (b >> 1) == 0 ? vr[j].x : (b >> 1) == 1 ? vr[j].y : (b >> 1) == 2 ? vr[j].z : vr[j].w;
                    a[j] = (_Float16)bf16_to_f32((uint16_t)((b & 1) ? (x >> 16) : (x & 0xFFFFu)));
                }
                o[b] = o[b] * alpha;
                o[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pb, o[b], 0, 0, 0);
            }
        }
    }
    lsum = xor32_sum(xor16_sum(lsum));
    // ---- partial of this split: m, l (G) and acc (G, 512) ------------------
    const long base = (long)r * split + sp;
    if (wave == 0 && kg == 0 && r16 < H) {
        m_part[base * ML_H + r16] = m;
        l_part[base * ML_H + r16] = lsum;
    }
    if (r16 < H) {
        float* ap = acc_part + (base * ML_H + r16) * ML_D + 128 * wave + 32 * kg;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            *reinterpret_cast<float4*>(ap + 8 * v) = make_float4(o[0][v], o[1][v], o[2][v], o[3][v]);
            *reinterpret_cast<float4*>(ap + 8 * v + 4) = make_float4(o[4][v], o[5][v], o[6][v], o[7][v]);
        }
    }
}

// LSE merge of the active splits (merge.py:105-152 rule) into o (R, H, 512)
// and lse (R, H).  Grid (H, R, 512 / (4 COLS) slices); 256 threads = COLS
// float4 columns x 256 / COLS split groups, each group's first PF partials
// loaded before anything waits, the rest in batches of PF, reduced in LDS.
// Sparse rows (tens of splits): COLS 32 (4 slices of 128 dims).  The dense
// comparator (hundreds of splits): COLS 8 (16 slices of 32 dims, 256
// workgroups per request instead of 64) and PF 8, so a 512-split row is
// two rounds of loads per thread instead of sixteen.
constexpr int MG_BLK = 256;

template <int COLS, int PF>
__global__ __launch_bounds__(MG_BLK) void mla_merge_kernel(
    const float* __restrict__ m_part, const float* __restrict__ l_part,
    const float* __restrict__ acc_part, const int* __restrict__ pcnt, int pt_cols,
    const int* __restrict__ seq_lens, int bt_cols,
    void* __restrict__ out, long o_sr, long o_sh, int out_f32,
    float* __restrict__ lse, long lse_sr, int split, int pps_min)
{
    const int h = blockIdx.x, r = blockIdx.y, zc = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // page count: the selection's (clamped to the table) or, with pcnt ==
    // nullptr, every page of the row (the dense comparator)
    const int cnt = pcnt ? min(pcnt[r], pt_cols) : min(cdiv(seq_lens[r], ML_PG), bt_cols);
    const int pps = max(cdiv(cnt, split), pps_min);
    const int n_act = cnt > 0 ? cdiv(cnt, pps) : 0;
    __shared__ float w_s[MD_MAX_SPLIT];
    __shared__ float red[MG_BLK / kWave];
    constexpr int MG_GRP = MG_BLK / COLS;
    __shared__ __attribute__((aligned(16))) float4 part[MG_GRP][COLS];
    const long rb = (long)r * split;
    const int c = tid % COLS, g = tid / COLS;
    const int d0 = 4 * COLS * zc + 4 * c;
    // the first PF partials of this thread's split group, loaded before any
    // wait (they do not depend on the weights)
    float4 pre[PF];
#pragma unroll
    for (int k = 0; k < PF; ++k) {
        const int s = g + k * MG_GRP;
        pre[k] = (s < split) ? *reinterpret_cast<const float4*>(acc_part + ((rb + s) * ML_H + h) * ML_D + d0)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // this thread's split (m, l) in the same round trip (clamped index;
    // masked by the active count below)
    const long ml0 = (rb + min(tid, split - 1)) * ML_H + h;
    const float m0 = m_part[ml0], l0 = l_part[ml0];
    const bool has0 = tid < n_act && l0 > 0.f;
    // M = max over live splits; weights; L = sum w l (fixed reduction tree)
    float mx = has0 ? m0 : -INFINITY;
    for (int s = tid + MG_BLK; s < n_act; s += MG_BLK) {
        const long i = (rb + s) * ML_H + h;
        if (l_part[i] > 0.f) mx = fmaxf(mx, m_part[i]);
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    lds_barrier();
    float M = red[0];
#pragma unroll
    for (int w = 1; w < MG_BLK / kWave; ++w) M = fmaxf(M, red[w]);
    lds_barrier();
    const float w0 = has0 ? __expf(m0 - M) : 0.f;
    if (tid < n_act) w_s[tid] = w0;
    float lp = has0 ? w0 * l0 : 0.f;
    for (int s = tid + MG_BLK; s < n_act; s += MG_BLK) {
        const long i = (rb + s) * ML_H + h;
        const float l = l_part[i];
        const float w = (l > 0.f) ? __expf(m_part[i] - M) : 0.f;
        w_s[s] = w;
        lp += w * l;
    }
    lp += row_ror<8>(lp); lp += row_ror<4>(lp); lp += row_ror<2>(lp); lp += row_ror<1>(lp);
    lp = xor32_sum(xor16_sum(lp));
    if (lane == 0) red[wave] = lp;
    lds_barrier();
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < MG_BLK / kWave; ++w) L += red[w];
    // acc over this slice: column c (4 dims), split group g
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    // every weight read issued before the first use (a guarded read per
    // partial was one LDS round trip each); inactive partials left out by
    // selects (their rows may be stale)
    float wk[PF];
#pragma unroll
    for (int k = 0; k < PF; ++k) wk[k] = w_s[min(g + k * MG_GRP, MD_MAX_SPLIT - 1)];
#pragma unroll
    for (int k = 0; k < PF; ++k) {
        const bool on = g + k * MG_GRP < n_act;
        acc.x = on ? acc.x + wk[k] * pre[k].x : acc.x;
        acc.y = on ? acc.y + wk[k] * pre[k].y : acc.y;
        acc.z = on ? acc.z + wk[k] * pre[k].z : acc.z;
        acc.w = on ? acc.w + wk[k] * pre[k].w : acc.w;
    }
    int s = g + PF * MG_GRP;
    for (; s + (PF - 1) * MG_GRP < n_act; s += PF * MG_GRP) {
        float4 a[PF];
        float w[PF];
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            a[k] = *reinterpret_cast<const float4*>(acc_part + ((rb + s + k * MG_GRP) * ML_H + h) * ML_D + d0);
            w[k] = w_s[s + k * MG_GRP];
        }
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            acc.x += w[k] * a[k].x; acc.y += w[k] * a[k].y; acc.z += w[k] * a[k].z; acc.w += w[k] * a[k].w;
        }
    }
    for (; s < n_act; s += MG_GRP) {
        const float4 a = *reinterpret_cast<const float4*>(acc_part + ((rb + s) * ML_H + h) * ML_D + d0);
        const float w = w_s[s];
        acc.x += w * a.x; acc.y += w * a.y; acc.z += w * a.z; acc.w += w * a.w;
    }
    part[g][c] = acc;
    lds_barrier();
    if (g == 0) {
        float4 o = part[0][c];
#pragma unroll
        for (int k = 1; k < MG_GRP; ++k) {
            const float4 x = part[k][c];
            o.x += x.x; o.y += x.y; o.z += x.z; o.w += x.w;
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        const float4 o4 = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
        if (out_f32) {
            *reinterpret_cast<float4*>(static_cast<float*>(out) + r * o_sr + h * o_sh + d0) = o4;
        } else {
            uint16_t* op = static_cast<uint16_t*>(out) + r * o_sr + h * o_sh + d0;
            *reinterpret_cast<uint2*>(op) = make_uint2((uint32_t)f32_to_bf16(o4.x) | ((uint32_t)f32_to_bf16(o4.y) << 16),
                                                       (uint32_t)f32_to_bf16(o4.z) | ((uint32_t)f32_to_bf16(o4.w) << 16));
        }
    }
    if (zc == 0 && tid == 0 && lse) lse[r * lse_sr + h] = L > 0.f ? M + __logf(L) : -INFINITY;
}

}  // namespace locks

using namespace locks;

extern "C" int32_t locks_mla_score(
    const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
    const uint8_t* v4, const uint16_t* vs, const int8_t* c8, const uint16_t* cs,
    const int8_t* mu8, const uint16_t* mus, const int8_t* rk8, const uint16_t* rks,
    const uint16_t* cache, int64_t c_stride_block,
    int64_t c_stride_tok, int32_t num_blocks, const int32_t* block_table, int64_t bt_stride,
    int32_t bt_cols, const int32_t* n_sel_hi, float* score, int64_t score_stride,
    int32_t max_pages, int32_t chunk, int32_t n_req, int32_t n_heads, int32_t kv_lora_rank,
    int32_t rope_dim, int32_t page, float scale, void* stream)
{
    LOCKS_REQUIRE(kv_lora_rank == ML_D && rope_dim == ML_DR && page == ML_PG,
                  "locks_mla_score: geometry (%d, %d, page %d) unsupported (this build: 512 + 64, page 16)",
                  kv_lora_rank, rope_dim, page);
    LOCKS_REQUIRE(n_heads >= 1 && n_heads <= ML_H, "locks_mla_score: n_heads=%d outside [1, %d]", n_heads, ML_H);
    LOCKS_REQUIRE(n_req >= 0 && num_blocks >= 1 && bt_cols >= 1 && max_pages >= 1,
                  "locks_mla_score: empty geometry");
    LOCKS_REQUIRE(chunk >= 2 && chunk % 2 == 0 && chunk <= ML_MAX_CHUNK,
                  "locks_mla_score: chunk %d must be even in [2, %d]", chunk, ML_MAX_CHUNK);
    LOCKS_REQUIRE(q_stride_head % 8 == 0 && q_stride_req % 8 == 0 && c_stride_tok % 8 == 0 &&
                  c_stride_block % 8 == 0, "locks_mla_score: strides must be multiples of 8 elements");
    LOCKS_REQUIRE((rk8 == nullptr) == (rks == nullptr),
                  "locks_mla_score: rk8 and rks must both be given (int8 RoPE summary) or both NULL");
    LOCKS_REQUIRE(q && v4 && vs && c8 && cs && mu8 && mus && (rk8 || cache) && block_table && n_sel_hi && score,
                  "locks_mla_score: null pointer argument");
    if (n_req == 0) return 0;
    const int Z = cdiv(max_pages, chunk);
#define LAUNCH_RQ(RQ)                                                                               \
    hipLaunchKernelGGL(mla_score_kernel<RQ>, dim3(Z, n_req), dim3(ML_BLK), (size_t)chunk * sizeof(int), (hipStream_t)stream, q, \
                       (long)q_stride_req, (long)q_stride_head, v4, vs, c8, cs, mu8, mus, rk8, rks,  \
                       cache, (long)c_stride_block, (long)c_stride_tok, num_blocks, block_table,     \
                       (long)bt_stride, bt_cols, n_sel_hi, score, (long)score_stride, max_pages,     \
                       n_heads, scale, chunk)
    if (rk8) LAUNCH_RQ(true);
    else LAUNCH_RQ(false);
#undef LAUNCH_RQ
    return check_launch("mla_score_kernel");
}

extern "C" int32_t locks_mla_build_rope(const uint16_t* cache, int64_t c_stride_block,
                                        int64_t c_stride_tok, int32_t num_blocks,
                                        const int32_t* blocks, int32_t n_blocks,
                                        const int32_t* n_blocks_dev, int8_t* rk8, uint16_t* rks,
                                        void* stream)
{
    LOCKS_REQUIRE(num_blocks >= 1 && n_blocks >= 0, "locks_mla_build_rope: bad geometry");
    LOCKS_REQUIRE(c_stride_tok % 8 == 0 && c_stride_block % 8 == 0,
                  "locks_mla_build_rope: strides must be multiples of 8 elements");
    LOCKS_REQUIRE(cache && blocks && rk8 && rks, "locks_mla_build_rope: null pointer argument");
    if (n_blocks == 0) return 0;
    hipLaunchKernelGGL(mla_rope_quant_kernel, dim3(cdiv(n_blocks, MR_WAVES)), dim3(MR_WAVES * kWave), 0,
                       (hipStream_t)stream, cache, (long)c_stride_block, (long)c_stride_tok, num_blocks,
                       blocks, n_blocks, n_blocks_dev, rk8, rks);
    return check_launch("mla_rope_quant_kernel");
}

extern "C" int32_t locks_mla_score_auto_chunk(int32_t n_req, int32_t max_pages) {
    // ~512 workgroups over all (request, page pair) units, whole pairs
    const long pairs = (long)cdiv(max_pages > 0 ? max_pages : 1, 2) * (n_req > 0 ? n_req : 1);
    long per_wg = (pairs + 511) / 512;
    if (per_wg < 1) per_wg = 1;
    if (per_wg > ML_MAX_CHUNK / 2) per_wg = ML_MAX_CHUNK / 2;
    return (int32_t)(2 * per_wg);
}

extern "C" int32_t locks_mla_decode_splitk(
    const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head, const uint16_t* cache,
    int64_t c_stride_block, int64_t c_stride_tok, int32_t num_blocks, const int32_t* block_table,
    int64_t bt_stride, int32_t bt_cols, const int32_t* page_table, int64_t pt_stride,
    int32_t pt_cols, const int32_t* page_cnt, const int32_t* seq_lens, float* m_part,
    float* l_part, float* acc_part, int32_t n_req, int32_t n_heads, int32_t kv_lora_rank,
    int32_t rope_dim, int32_t page, int32_t split, int32_t pps_min, float scale, void* stream)
{
    LOCKS_REQUIRE(kv_lora_rank == ML_D && rope_dim == ML_DR && page == ML_PG,
                  "locks_mla_decode_splitk: geometry (%d, %d, page %d) unsupported (this build: 512 + 64, page 16)",
                  kv_lora_rank, rope_dim, page);
    LOCKS_REQUIRE(n_heads >= 1 && n_heads <= ML_H, "locks_mla_decode_splitk: n_heads=%d outside [1, %d]",
                  n_heads, ML_H);
    LOCKS_REQUIRE(split >= 1 && split <= MD_MAX_SPLIT && pps_min >= 1,
                  "locks_mla_decode_splitk: split=%d pps_min=%d (split in [1, %d])", split, pps_min, MD_MAX_SPLIT);
    LOCKS_REQUIRE(q_stride_head % 8 == 0 && q_stride_req % 8 == 0 && c_stride_tok % 8 == 0 &&
                  c_stride_block % 8 == 0, "locks_mla_decode_splitk: strides must be multiples of 8 elements");
    LOCKS_REQUIRE(n_req >= 0 && num_blocks >= 1 && bt_cols >= 1 && pt_cols >= 1,
                  "locks_mla_decode_splitk: empty geometry");
    LOCKS_REQUIRE(q && cache && block_table && page_table && page_cnt && seq_lens && m_part && l_part && acc_part,
                  "locks_mla_decode_splitk: null pointer argument");
    if (n_req == 0) return 0;
    hipLaunchKernelGGL((mla_decode_split_kernel<false, 2, 0>), dim3(split, n_req), dim3(ML_BLK), 0, (hipStream_t)stream,
                       q, (long)q_stride_req, (long)q_stride_head, cache, (long)c_stride_block,
                       (long)c_stride_tok, num_blocks, block_table, (long)bt_stride, bt_cols,
                       page_table, (long)pt_stride, pt_cols, page_cnt, seq_lens, m_part, l_part,
                       acc_part, n_heads, split, pps_min, scale);
    return check_launch("mla_decode_split_kernel");
}

extern "C" int32_t locks_mla_decode_merge(
    const float* m_part, const float* l_part, const float* acc_part, const int32_t* page_cnt,
    int32_t pt_cols, void* out, int64_t out_stride_req, int64_t out_stride_head, int32_t out_is_f32,
    float* lse, int64_t lse_stride_req, int32_t n_req, int32_t n_heads, int32_t kv_lora_rank,
    int32_t split, int32_t pps_min, void* stream)
{
    LOCKS_REQUIRE(kv_lora_rank == ML_D, "locks_mla_decode_merge: kv_lora_rank %d unsupported (512)", kv_lora_rank);
    LOCKS_REQUIRE(n_heads >= 1 && n_heads <= ML_H, "locks_mla_decode_merge: n_heads=%d outside [1, %d]",
                  n_heads, ML_H);
    LOCKS_REQUIRE(split >= 1 && split <= MD_MAX_SPLIT && pps_min >= 1, "locks_mla_decode_merge: bad split");
    LOCKS_REQUIRE(out_stride_req % 4 == 0 && out_stride_head % 4 == 0,
                  "locks_mla_decode_merge: out strides must be multiples of 4 elements");
    LOCKS_REQUIRE(m_part && l_part && acc_part && page_cnt && out, "locks_mla_decode_merge: null pointer argument");
    if (n_req == 0) return 0;
    hipLaunchKernelGGL((mla_merge_kernel<32, 4>), dim3(n_heads, n_req, ML_D / 128), dim3(MG_BLK), 0, (hipStream_t)stream,
                       m_part, l_part, acc_part, page_cnt, pt_cols, nullptr, 1, out, (long)out_stride_req,
                       (long)out_stride_head, out_is_f32, lse, (long)lse_stride_req, split, pps_min);
    return check_launch("mla_merge_kernel");
}

#ifndef LOCKS_MLA_DENSE_NST
#define LOCKS_MLA_DENSE_NST 3
#endif
extern "C" int32_t locks_mla_decode_dense(
    const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head, const uint16_t* cache,
    int64_t c_stride_block, int64_t c_stride_tok, int32_t num_blocks, const int32_t* block_table,
    int64_t bt_stride, int32_t bt_cols, const int32_t* seq_lens, float* m_part, float* l_part,
    float* acc_part, void* out, int64_t out_stride_req, int64_t out_stride_head, int32_t out_is_f32,
    float* lse, int64_t lse_stride_req, int32_t n_req, int32_t n_heads, int32_t kv_lora_rank,
    int32_t rope_dim, int32_t page, int32_t split, float scale, void* stream)
{
    LOCKS_REQUIRE(kv_lora_rank == ML_D && rope_dim == ML_DR && page == ML_PG,
                  "locks_mla_decode_dense: geometry (%d, %d, page %d) unsupported (this build: 512 + 64, page 16)",
                  kv_lora_rank, rope_dim, page);
    LOCKS_REQUIRE(n_heads >= 1 && n_heads <= ML_H, "locks_mla_decode_dense: n_heads=%d outside [1, %d]",
                  n_heads, ML_H);
    LOCKS_REQUIRE(split >= 1 && split <= MD_MAX_SPLIT, "locks_mla_decode_dense: split=%d outside [1, %d]",
                  split, MD_MAX_SPLIT);
    LOCKS_REQUIRE(q_stride_head % 8 == 0 && q_stride_req % 8 == 0 && c_stride_tok % 8 == 0 &&
                  c_stride_block % 8 == 0, "locks_mla_decode_dense: strides must be multiples of 8 elements");
    LOCKS_REQUIRE(out_stride_req % 4 == 0 && out_stride_head % 4 == 0,
                  "locks_mla_decode_dense: out strides must be multiples of 4 elements");
    LOCKS_REQUIRE(n_req >= 0 && num_blocks >= 1 && bt_cols >= 1, "locks_mla_decode_dense: empty geometry");
    LOCKS_REQUIRE(q && cache && block_table && seq_lens && m_part && l_part && acc_part && out,
                  "locks_mla_decode_dense: null pointer argument");
    if (n_req == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL((mla_decode_split_kernel<true, LOCKS_MLA_DENSE_NST, CPOL_NT_MLA>), dim3(split, n_req),
                       dim3(ML_BLK), 0, st, q, (long)q_stride_req, (long)q_stride_head, cache,
                       (long)c_stride_block, (long)c_stride_tok, num_blocks, block_table, (long)bt_stride,
                       bt_cols, nullptr, 0L, 1, nullptr, seq_lens, m_part, l_part, acc_part, n_heads,
                       split, 1, scale);
    if (int rc = check_launch("mla_decode_split_kernel<dense>")) return rc;
    hipLaunchKernelGGL((mla_merge_kernel<8, 8>), dim3(n_heads, n_req, ML_D / 32), dim3(MG_BLK), 0, st,
                       m_part, l_part, acc_part, nullptr, 1, seq_lens, bt_cols, out, (long)out_stride_req,
                       (long)out_stride_head, out_is_f32, lse, (long)lse_stride_req, split, 1);
    return check_launch("mla_merge_kernel");
}
