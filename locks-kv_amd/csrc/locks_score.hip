// rki4 page scorer for gfx950 (CDNA4).
//
// Computes, for every selectable logical page p < n_sel_hi[r] of request r
// and kv head kh, the per-query-head page log-sum-exp estimate from the
// packed rank-8 int4 summary (reference: selection/rki4_score_cuda.py:653-722,
// fp32 twin selection/rki4_score_torch.py:111-160):
//
//   q8 = rint(q / qs), qs = max(|q|_inf, 1e-8) / 127           (per head)
//   qt[g][c]  = (sum_d V4[c][d] * q8[g][d]) * qs[g] * vs[c]      c < 8
//   mud[g]    = (sum_d mu8[d]   * q8[g][d]) * qs[g] * mus
//   tok[g][t] = s * (cs[t] * sum_c c8[t][c] * qt[g][c] + mud[g])   t < 16
//   score_h[g][p] = LSE_t tok[g][t]
//
// MI355X mapping.  One workgroup = 4 waves owns a contiguous chunk of pages
// of one (request, kv head); a wave scores 8-page units:
//   * the int4 x int8 projection of the whole GQA group runs on the matrix
//     core: v_mfma_i32_16x16x64_i8 with A = 16 packed-V rows (2 pages x 8
//     basis columns; 4 pages x 4 columns when G <= 4) and B = int8 q (column
//     = head).  Each int4 nibble is moved to the high half of its byte (a
//     shift and two ANDs per 8 values), so the operand is 16 V as int8, no
//     sign extension; the 1/16 rides on the column scale;
//   * mu . q8 uses the same MFMA with A = the int8 q rows and B = one mu row
//     per column (page);
//   * the per-token reconstruction sum_c c8[t][c] qt[g][c] is a 16x8 by
//     8xG product per page: v_mfma_f32_16x16x4_f32 with pages packed side by
//     side when 4 < G < 16 (block-diagonal B); for G <= 4,
//     v_mfma_f32_4x4x1_16b_f32 with one 4x4 block per (page, 4-token quad),
//     so no block-diagonal zeros are multiplied.  The VALU only does the
//     cs/mu epilogue and the 16-token LSE.
// Summary bytes are read exactly once: each unit's 8 records (or the six
// separate slabs' rows) are DMA'd through the block table into a per-wave
// LDS stage, one unit ahead, and with one request the units of a wave are
// software-pipelined (the next unit's projection interleaves with this
// unit's token stage).  Per-workgroup page maxima are published to `pmax`
// so the selector can form the per-head max without re-reading score_h.
#include "locks_common.h"
#include "locks_hip.h"

namespace locks {

constexpr int SC_RNK = 8;     // summary rank
constexpr int SC_TILE = 8;    // pages per wave tile
constexpr int SC_WAVES = 4;
constexpr int SC_BLOCK = SC_WAVES * kWave;
constexpr int SC_MAX_CHUNK = 1024;          // pages per workgroup, upper bound
constexpr int SC_STAGE_F = 4096;            // STG: floats of score_h staged per workgroup (16 KB)
constexpr int SC_CPOL_NT = 2;                // buffer-load cache policy: non-temporal

// Per-geometry layout (head_dim D in {64, 128, 256}, page PG in {16, 32, 64}).
// A summary row (one page, one kv head) holds, in this order (the
// reference's AoS record, selection/rki4_state.py:93-110, 198-219):
//   v4  8 columns x D/2 B   int4 basis (column-major, low nibble = even d)
//   mu  D B                 centroid
//   c8  PG tokens x 8 B     coefficients
//   cs  PG x bf16           token scales
//   vs  8 x bf16            column scales
//   mus bf16                centroid scale (+ pad)
// i.e. 5D + 10PG + 18 bytes rounded up to 64 when the state packs the fields
// together (RS; 832 B at D = 128, PG = 16).  One wave's unit is 8 such rows;
// all fields but mus (RB = 5D + 10PG + 16 bytes per row) are DMA'd as ONE
// byte stream (global_load_lds_dwordx4: lane L of
// instruction i fetches stream chunk 64 i + L into LDS byte 16 (64 i + L))
// into a row-major LDS stage, so each instruction reads ~1 KB of consecutive
// row bytes -- measured 16-22 % faster than field-wise DMA of the same rows.
// The centroid scale goes to a VGPR.  With separate slabs (the reference's
// layout) each lane picks its chunk's slab instead; the stage is the same.
template <int D, int PG>
struct ScGeom {
    static_assert(D == 64 || D == 128 || D == 256, "head_dim 64, 128 or 256");
    static_assert(PG == 16 || PG == 32 || PG == 64, "page 16, 32 or 64");
    static constexpr int NWIN = D / 64;                // 16-d windows per lane (projection MFMAs)
    static constexpr int NTB = PG / 16;                // 16-token blocks per page
    static constexpr int O_MU = 4 * D;                 // field offsets inside a row
    static constexpr int O_C8 = O_MU + D;
    static constexpr int O_CS = O_C8 + 8 * PG;
    static constexpr int O_VS = O_CS + 2 * PG;
    static constexpr int RB = O_VS + 16;               // stage row bytes (all fields but mus)
    static constexpr int CPR = RB / 16;                // 16-B chunks per stage row
    static constexpr int NCK = SC_TILE * CPR;          // chunks per unit
    static constexpr int NDI = (NCK + 63) / 64;        // DMA instructions per unit
    static constexpr int ST_BYTES = SC_TILE * RB;
    static constexpr int QROW = D + 16;                // padded int8 q row
};

typedef __attribute__((address_space(3))) void* sc_lds_ptr;

// One lane's sources for one unit: per DMA instruction a byte offset from
// the v4 base (packed rows) or a full address (separate slabs), and the
// centroid scale's offset.
template <int NDI, bool PK>
struct ScUnitSrc { uint32_t off[PK ? NDI : 1]; const uint8_t* addr[PK ? 1 : NDI]; uint32_t mus; };

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    return (uint32_t)(uint8_t)a | ((uint32_t)(uint8_t)b << 8) |
           ((uint32_t)(uint8_t)c << 16) | ((uint32_t)(uint8_t)d << 24);
}

template <int GW, int D = 128, int PG = 16, bool PK = true, bool PIPE = true, bool STG = false>
__global__ __launch_bounds__(SC_BLOCK) void rki4_score_kernel(
    const uint16_t* __restrict__ q, long q_sr, long q_sh, SlabRows S, int NB, const int* __restrict__ bt, long bt_sr, int bt_cols,
    const int* __restrict__ nsh, float* __restrict__ score_h, int MP,
    float* __restrict__ pmax, int n_kv, int G, float sm_scale, int chunk)
{
    using GM = ScGeom<D, PG>;
    constexpr int PPM = 16 / GW;            // pages per token-stage MFMA
    constexpr int NGRP = SC_TILE / PPM;     // token-stage groups per tile
    constexpr int NWIN = GM::NWIN, NTB = GM::NTB, SC_QROW = GM::QROW;
    constexpr int O_C8 = GM::O_C8, O_MU = GM::O_MU, O_CS = GM::O_CS, O_VS = GM::O_VS, RB = GM::RB;
    constexpr int CPR = GM::CPR, NCK = GM::NCK, NDI = GM::NDI;
    constexpr int QDL = D <= 128 ? 8 : 16;  // q dims per lane in the quantize step
    constexpr int LPH = D / QDL;            // q lanes per head (8 or 16: one DPP row group)
    const int z = blockIdx.x, h = blockIdx.y, r = blockIdx.z;   // page chunk, kv head, request
    const int Z = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int P = min(nsh[r], MP);          // never score past the score_h row
    const int c0 = z * chunk;
    const int c1 = min(c0 + chunk, P);
    float* pm_out = pmax + ((long)r * n_kv + h) * 16 * Z + z;     // head-major: pm_out[g * Z]

    if (c0 >= P) {                          // no page of this chunk is scored
        if (tid < 16) pm_out[(long)tid * Z] = -INFINITY;
        return;
    }

    __shared__ __attribute__((aligned(16))) float qsp[16];
    // two stages per wave, alternating between units, as separate LDS
    // objects: the next unit's DMA never shares an object with the current
    // unit's reads (the compiler's memory-counter tracking would otherwise
    // wait for the DMA before every read)
    __shared__ __attribute__((aligned(16))) uint8_t sa_l[SC_WAVES][GM::ST_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t sb_l[SC_WAVES][GM::ST_BYTES];
    __shared__ uint32_t wmax[16];
    // STG: the workgroup's scores [head][page of the chunk], written out
    // coalesced after the last unit.  Stored straight to score_h, each unit's
    // scattered stores (8 pages x G per wave) sat in the vector-memory counter
    // ahead of the next unit's record DMA, and the wait for that DMA waited
    // for them too (GLM 1M scorer 28.5 -> 26 us with the stores left out).  A
    // static object of its own: the compiler sees it is not a DMA target and
    // does not wait for the DMA before writing it.
    // (rows padded by one float: at a 256-page chunk the heads of one store
    // would otherwise all hit one bank)
    __shared__ __attribute__((aligned(16))) float sc_l[STG ? SC_STAGE_F + 16 : 1];
    // PIPE: centroid terms mud[page][head] of a wave's last two units (rows
    // 8-15: idle lanes); otherwise they go to the unit's consumed stage rows
    __shared__ __attribute__((aligned(16))) float mud_l[PIPE ? SC_WAVES : 1][2][PIPE ? 16 * 16 : 4];
    // dynamic LDS: slab rows (block x n_kv + kv head) of the chunk
    extern __shared__ __attribute__((aligned(16))) int dyn_l[];
    int* bt_l = dyn_l;
    // int8 q rows of this kv head's G query heads (+16 zero rows) live in the
    // second stages until the q operands are built: no DMA reaches them
    // before the first unit, and the workgroup fits three to a CU
    static_assert((16 + 16) * SC_QROW <= SC_WAVES * GM::ST_BYTES, "q rows fit the second stages");
    int8_t (*q8s)[SC_QROW] = reinterpret_cast<int8_t (*)[SC_QROW]>(&sb_l[0][0]);

    // ---- prologue: q rows and block ids are fetched together; the first
    // unit's summary loads are issued before q is quantized, so the
    // quantization overlaps them.
    // q: LPH consecutive lanes per head, QDL dims (one or two 16-byte loads)
    // per lane (G <= 16 heads x LPH lanes <= 256 threads)
    // Unconditional loads (threads past the group re-read its last head and
    // are never stored): a guarded load would make the compiler wait for it
    // at the branch join, before the block ids below are even requested.
    const int qg = tid / LPH;                                 // this thread's head in the group
    const uint4* qp = reinterpret_cast<const uint4*>(q + (long)r * q_sr + (long)(h * G + min(qg, G - 1)) * q_sh + (tid % LPH) * QDL);
    const uint4 qa0 = qp[0], qa1 = (QDL == 16) ? qp[1] : qa0;
    for (int i = tid; i < c1 - c0; i += SC_BLOCK) {
        const int b = bt[(long)r * bt_sr + min(c0 + i, bt_cols - 1)];
        bt_l[i] = min(max(b, 0), NB - 1) * n_kv + h;           // slab row of (block, kv head)
    }
    if (tid < 16) {
        wmax[tid] = 0x007FFFFFu;                               // f2u(-inf)
        qsp[tid] = 0.f;
    }
    for (int i = tid; i < 16 * SC_QROW / 4; i += SC_BLOCK)
        reinterpret_cast<int*>(&q8s[G][0])[i] = 0;             // zero rows after the last head
    __syncthreads();

    const int r16 = lane & 15, kg = lane >> 4;
    const int jcol = lane & 15;
    const int psub_l = jcol / GW;            // page slot of this lane's column
    const int g_l = jcol % GW;               // head of this lane's column
    // G <= 4: the token stage runs on v_mfma_f32_4x4x1_16b_f32, 16 blocks of
    // (page, 4-token quad) x 4 heads, instead of block-diagonal 16x16x4
    // products three quarters zero
    constexpr bool TK4 = (GW == 4);
    const uint32_t MH = 0xF0F0F0F0u;
    const int n_tiles = cdiv(c1 - c0, SC_TILE);
    const int n_units = n_tiles;             // (8-page tile) units of the chunk

    // Each (8-page tile, kv head) unit's rows are DMA'd straight from the
    // slabs into this wave's LDS stage (no VGPR round trip), non-temporally:
    // every row is read once.  Consecutive units are the kv heads of one
    // tile, whose rows are adjacent.
    const auto rs_mus = __builtin_amdgcn_make_buffer_rsrc(S.mus, 0, -1, 0x00020000);
    // row strides (bytes) of the slabs: offsets below stay under 2^32
    const uint32_t sv4 = (uint32_t)S.sv4, svs = (uint32_t)S.svs, sc8 = (uint32_t)S.sc8,
                   scs = (uint32_t)S.scs, smu = (uint32_t)S.smu, smus = (uint32_t)S.smus;
    uint32_t fmus = 0;                               // centroid scale of page lane & 15 (lanes & 15 < 8)
    // Every lane's sources of one unit, read from the slab rows in LDS while
    // no DMA is outstanding (an LDS read issued behind a DMA waits for it)
    // and pinned in registers before the first DMA of the unit.
    using UnitSrc = ScUnitSrc<NDI, PK>;
    auto unit_src = [&](int u) -> UnitSrc {
        const int p0 = u * SC_TILE;
        const int last = min(SC_TILE, c1 - c0 - p0) - 1;   // tail pages repeat the last one
        auto row = [&](int i) -> uint32_t { return (uint32_t)bt_l[p0 + min(i, last)]; };
        UnitSrc f;
        uint32_t w[NDI];                             // all block-id reads first, then the math
#pragma unroll
        for (int i = 0; i < NDI; ++i) w[i] = row(min(64 * i + lane, NCK - 1) / CPR);
#pragma unroll
        for (int i = 0; i < NDI; ++i) {
            const int sk = min(64 * i + lane, NCK - 1);     // stream chunk (lanes past the end: idle)
            const int o = 16 * (sk % CPR);                  // byte in the row
            if constexpr (PK) {
                f.off[i] = w[i] * sv4 + o;
            } else {
                const uint8_t* a;
                if (o < O_MU) a = S.v4 + (size_t)w[i] * sv4 + o;
                else if (o < O_C8) a = S.mu + (size_t)w[i] * smu + (o - O_MU);
                else if (o < O_CS) a = S.c8 + (size_t)w[i] * sc8 + (o - O_C8);
                else if (o < O_VS) a = S.cs + (size_t)w[i] * scs + (o - O_CS);
                else a = S.vs + (size_t)w[i] * svs;
                f.addr[i] = a;
            }
        }
        f.mus = row(lane & 7) * smus;
#pragma unroll
        for (int i = 0; i < (PK ? NDI : 1); ++i) asm volatile("" :: "v"(f.off[i]));
#pragma unroll
        for (int i = 0; i < (PK ? 1 : NDI); ++i) asm volatile("" :: "v"(f.addr[i]));
        asm volatile("" :: "v"(f.mus));
        return f;
    };
    auto issue = [&](const UnitSrc& f, uint8_t* st) {
#pragma unroll
        for (int i = 0; i < NDI; ++i) {
            // copied out first: a member of f inside the builtin's arguments
            // makes the host pass drop the kernel stub
            const uint8_t* src;
            if constexpr (PK) { const uint32_t o = f.off[i]; src = S.v4 + o; }
            else src = f.addr[i];
            if (NCK % 64 == 0 || i < NDI - 1 || lane < NCK - 64 * (NDI - 1))
                __builtin_amdgcn_global_load_lds(src, (sc_lds_ptr)(st + 1024 * i), 16, 0, SC_CPOL_NT);
        }
        const uint32_t om = f.mus;
        if ((lane & 15) < 8)
            fmus = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs_mus, (int)om, 0, 0);
    };
    __builtin_amdgcn_s_waitcnt(0x0070);      // q rows resident before the unit loads queue
    if (wave < n_units) issue(unit_src(wave), sa_l[wave]);

    // ---- quantize q (the first unit's loads are in flight) --------------
    // q8 = rint(q / qs) with the correctly rounded quotient: q * (1 / qs) is
    // within 2 ulp of it, which decides the rounding unless the product lies
    // within 2^-15 of a half-integer; those (rare) lanes redo the division.
    const float s2 = sm_scale * 1.4426950408889634f;           // tokens in log2 units
    if (tid < G * LPH) {                                      // G heads x LPH lanes
        const int c = tid, hq = qg;
        const uint32_t w[8] = {qa0.x, qa0.y, qa0.z, qa0.w, qa1.x, qa1.y, qa1.z, qa1.w};
        float f[QDL];
#pragma unroll
        for (int k = 0; k < QDL / 2; ++k) { f[2 * k] = bf16lo(w[k]); f[2 * k + 1] = bf16hi(w[k]); }
        float am = 0.f;
#pragma unroll
        for (int k = 0; k < QDL; ++k) am = fmaxf(am, fabsf(f[k]));
        // max over the head's LPH lanes (aligned groups of 8 or 16) by DPP:
        // quad swaps, then the half-row and (16) row mirrors
        am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0xB1, 0xF, 0xF, false)));
        am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0x4E, 0xF, 0xF, false)));
        am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0x141, 0xF, 0xF, false)));
        if constexpr (LPH == 16)
            am = fmaxf(am, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(am), 0x140, 0xF, 0xF, false)));
        const float qs = fmaxf(am, 1e-8f) / 127.f;
        const float inv = 1.f / qs;
        int iq[QDL];
        bool near = false;
#pragma unroll
        for (int k = 0; k < QDL; ++k) {
            const float y = f[k] * inv;
            const float ry = rintf(y);
            near |= fabsf(fabsf(y - ry) - 0.5f) < 0x1p-15f;
            iq[k] = (int)ry;
        }
        if (__builtin_expect(__ballot(near) != 0ull, 0)) {
            if (near) {
#pragma unroll
                for (int k = 0; k < QDL; ++k) iq[k] = (int)rintf(__fdiv_rn(f[k], qs));
            }
        }
        int8_t* qrow = &q8s[hq][(c % LPH) * QDL];
        *reinterpret_cast<uint2*>(qrow) = make_uint2(pack4_i8(iq[0], iq[1], iq[2], iq[3]), pack4_i8(iq[4], iq[5], iq[6], iq[7]));
        if constexpr (QDL == 16)
            *reinterpret_cast<uint2*>(qrow + 8) = make_uint2(pack4_i8(iq[8], iq[9], iq[10], iq[11]), pack4_i8(iq[12], iq[13], iq[14], iq[15]));
        if (c % LPH == 0) qsp[hq] = qs * s2;
    }
    // barriers on the q rows while the first unit's DMA is in flight: the
    // compiler's LDS fences count a pending LDS DMA as an LDS write and would
    // wait for it, so the LDS completion wait and the barrier are explicit
    // (the asm a compiler memory barrier)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // int8 q rows of this kv head's GQA group as matrix-core operands (the
    // same for every unit of the workgroup):
    // Bq = projection B (column j <-> head j % GW, replicated over the
    // GW-wide page slots), Amu = centroid A (row <-> head, zero padded)
    v4i Bq[NWIN], Amu[NWIN];
    {
        // lane group kg covers d in [kg D / 4, (kg + 1) D / 4): NWIN windows of 16
        const int gq = r16 % GW;
        const int rowq = (gq < G) ? gq : G;                   // G.. = zero rows
        const int rowm = (r16 < G) ? r16 : G;
#pragma unroll
        for (int w = 0; w < NWIN; ++w) {
            const uint4 n0 = *reinterpret_cast<const uint4*>(&q8s[rowq][kg * (D / 4) + 16 * w]);
            const uint4 m0 = *reinterpret_cast<const uint4*>(&q8s[rowm][kg * (D / 4) + 16 * w]);
            Amu[w] = v4i{(int)m0.x, (int)m0.y, (int)m0.z, (int)m0.w};
            // V operand order inside a 16-d window: even d (low nibbles), then odd d
            Bq[w] = v4i{(int)__builtin_amdgcn_perm(n0.y, n0.x, 0x06040200u), (int)__builtin_amdgcn_perm(n0.w, n0.z, 0x06040200u),
                        (int)__builtin_amdgcn_perm(n0.y, n0.x, 0x07050301u), (int)__builtin_amdgcn_perm(n0.w, n0.z, 0x07050301u)};
        }
    }
    const float4 qsl = *reinterpret_cast<const float4*>(&qsp[4 * kg]);   // rows 4kg.. (mud)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // q rows consumed: the second stages are free
    // column head's q scale x 1/16 (the nibble shift), zeroed where the
    // token stage's block-diagonal B has no entry for this lane's column:
    // qt of page p feeds page slot p % PPM only (TK4: no zeros, every lane
    // group's qt belongs to its own block's page)
    float qsjm[PPM];
    {
        const float qsj = qsp[r16 % GW] * 0.0625f;
#pragma unroll
        for (int ps = 0; ps < PPM; ++ps) qsjm[ps] = (TK4 || psub_l == ps) ? qsj : 0.f;
    }

    float wrun = -INFINITY;                          // running per-head max of this lane's column
    // Software pipeline over a wave's units.  front(u) waits for unit u's
    // rows, reads every operand of the unit from its stage into registers
    // (packed V, column scales, centroid, and the token stage's coefficients
    // and token scales), issues the next unit's DMA, and runs the projection
    // and centroid MFMAs; back(u) runs the token stage, the LSE and the
    // stores from those registers and the unit's centroid terms.  A wave
    // runs front(u + 4) before back(u): the two chains are independent and
    // share one basic block, so the scheduler interleaves the projection of
    // one unit with the token MFMAs and exponentials of the one before.  No
    // stage holds live data after its front, so two stages per wave still
    // suffice; the centroid terms mud[page][head] go to a per-wave buffer of
    // two slots (rows 8-15 of a slot take the idle lanes' stores).
    // Without PIPE (grids of three workgroups per CU, which the pipeline's
    // registers and buffer do not fit) each unit runs front then back, and
    // mud goes into the first 64 B of each page's stage row (packed V,
    // consumed by then).
    constexpr int MUD_RS = PIPE ? 16 : RB / 4;                 // mud row stride (floats)
    struct Carry {
        float qt[4][4];
        uint2 c8w[TK4 ? 2 : 1][NTB];              // TK4: 8 coefficients of (page 4 gi + kg, token)
        uint32_t tw[TK4 ? 2 : SC_TILE][NTB];      // TK4: token scale bits; else cw | cs << 16
        int p0, nvalid;
        UnitSrc nf;                               // next unit's DMA sources
        bool more;
    };
    // Without STG a unit's scores are stored after the NEXT unit's record
    // wait: stored at once, they sat in the vector-memory counter behind the
    // next record DMA, and that unit's wait (vmcnt(0)) waited for them too
    // (ragged GLM batch: scorer 21.7 -> 21.1 us, step 1.830 -> 1.816 ms).
    constexpr int NPEND = STG ? 1 : (TK4 ? 1 : (NGRP + 3) / 4);
    float pend_v[NPEND];
    long pend_i[NPEND];
    bool pend_ok[NPEND];
#pragma unroll
    for (int k = 0; k < NPEND; ++k) { pend_v[k] = 0.f; pend_i[k] = 0; pend_ok[k] = false; }
    auto flush_pend = [&]() {
        if constexpr (STG) return;
#pragma unroll
        for (int k = 0; k < NPEND; ++k) {
            if (pend_ok[k]) score_h[pend_i[k]] = pend_v[k];
            pend_ok[k] = false;
        }
    };
    auto put_score = [&](int k, long idx, float v, bool ok) {
        if constexpr (STG) {
            (void)k; (void)idx; (void)v; (void)ok;
        } else {
            pend_v[k] = v; pend_i[k] = idx; pend_ok[k] = ok;
        }
    };
    auto front = [&](int u, uint8_t* st, uint8_t* st_next, float* mud) -> Carry {
        __builtin_amdgcn_s_waitcnt(0x0070);          // this unit's rows have landed in the stage
        flush_pend();                                // the previous unit's scores
        wave_lds_sync();
        const float musf = ((lane & 15) < 8) ? bf16lo(fmus) : 0.f;   // before the next unit's load
        Carry c;
        c.more = u + SC_WAVES < n_units;
        if (c.more) c.nf = unit_src(u + SC_WAVES);
        c.p0 = c0 + u * SC_TILE;
        c.nvalid = min(SC_TILE, c1 - c.p0);

        wave_lds_sync();

        // ---- projection: qt (8 basis columns x GQA group) per page -------
        // One MFMA pair per 2 pages: A = the 16 packed-V rows of the pair,
        // ordered so that row 4a + b holds (page 2pp + (b & 1), column
        // 2a + (b >> 1)); B = int8 q.  The result lands in lane (kg, j) as
        // qt[pp][v] = qt[head j % GW][page 2pp + (v & 1)][column 2kg + (v >> 1)],
        // which is exactly the B operand the token stage needs (its k-slot
        // kg, step hh reads column 2kg + hh), so qt never goes through LDS.
        // TK4: MFMA pp covers pages 4 (pp >> 1) .. + 3 x columns 4 (pp & 1) ..
        // + 3 (row 4a + b <-> page 4 (pp >> 1) + a, column 4 (pp & 1) + b), so
        // lane group kg ends with all 8 columns of page 4 gi + kg, the B
        // operand of its 4x4 blocks.
        const int i_pg = TK4 ? (r16 >> 2) : (r16 & 1);
        const int i_c = TK4 ? (r16 & 3) : 2 * (r16 >> 2) + ((r16 >> 1) & 1);
        auto pr_page = [&](int pp, int i) { return TK4 ? 4 * (pp >> 1) + i : 2 * pp + i; };
        auto pr_col = [&](int pp, int i) { return TK4 ? 4 * (pp & 1) + i : i; };
        // lane group kg reads D / 8 packed bytes (d in [kg D / 4, (kg + 1) D / 4))
        uint32_t vv[4][D / 32];
        float2 vsf[4][2];
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
            const uint8_t* rp = st + pr_page(pp, i_pg) * RB + pr_col(pp, i_c) * (D / 2) + kg * (D / 8);
            if constexpr (D == 64) {
                const uint2 x = *reinterpret_cast<const uint2*>(rp);
                vv[pp][0] = x.x; vv[pp][1] = x.y;
            } else {
#pragma unroll
                for (int k = 0; k < D / 128; ++k) {
                    const uint4 x = *reinterpret_cast<const uint4*>(rp + 16 * k);
                    vv[pp][4 * k] = x.x; vv[pp][4 * k + 1] = x.y; vv[pp][4 * k + 2] = x.z; vv[pp][4 * k + 3] = x.w;
                }
            }
            if constexpr (TK4) {                    // column scales 4 (pp & 1) .. + 3 of page 4 (pp >> 1) + kg
                const uint2 w = *reinterpret_cast<const uint2*>(st + pr_page(pp, kg) * RB + O_VS + 8 * (pp & 1));
                vsf[pp][0] = make_float2(bf16lo(w.x), bf16hi(w.x));
                vsf[pp][1] = make_float2(bf16lo(w.y), bf16hi(w.y));
            } else {
#pragma unroll
                for (int pg = 0; pg < 2; ++pg) {    // column scales (2kg, 2kg+1) of page 2pp+pg
                    const uint32_t w = *reinterpret_cast<const uint32_t*>(st + (2 * pp + pg) * RB + O_VS + kg * 4);
                    vsf[pp][pg] = make_float2(bf16lo(w), bf16hi(w));
                }
            }
        }
        v4i mu[NWIN];
#pragma unroll
        for (int w = 0; w < NWIN; ++w) mu[w] = v4i{0, 0, 0, 0};
        if ((lane & 15) < 8) {
            const int pg = lane & 15;
#pragma unroll
            for (int w = 0; w < NWIN; ++w)
                mu[w] = *reinterpret_cast<const v4i*>(st + pg * RB + O_MU + kg * (D / 4) + 16 * w);
        }
        // token-stage operands: coefficients and token scales of the lane's
        // token row (16 tb + r16)
#pragma unroll
        for (int tb = 0; tb < NTB; ++tb) {
            if constexpr (TK4) {
#pragma unroll
                for (int gi = 0; gi < 2; ++gi) {
                    const uint8_t* rp = st + (4 * gi + kg) * RB;
                    c.c8w[gi][tb] = *reinterpret_cast<const uint2*>(rp + O_C8 + (16 * tb + r16) * 8);
                    c.tw[gi][tb] = *reinterpret_cast<const uint16_t*>(rp + O_CS + (16 * tb + r16) * 2);
                }
            } else {
#pragma unroll
                for (int page = 0; page < SC_TILE; ++page) {
                    const uint8_t* rp = st + page * RB;
                    const uint32_t cw = *reinterpret_cast<const uint16_t*>(rp + O_C8 + (16 * tb + r16) * 8 + 2 * kg);
                    const uint32_t cs = *reinterpret_cast<const uint16_t*>(rp + O_CS + (16 * tb + r16) * 2);
                    c.tw[page][tb] = cw | (cs << 16);
                }
            }
        }
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
            // signed nibbles moved to the high half of each byte: 16 * V as int8
            v4i acc = {0, 0, 0, 0};
#pragma unroll
            for (int w = 0; w < NWIN; ++w) {
                const uint32_t w0 = vv[pp][2 * w], w1 = vv[pp][2 * w + 1];
                const v4i a = {(int)((w0 << 4) & MH), (int)((w1 << 4) & MH), (int)(w0 & MH), (int)(w1 & MH)};
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, Bq[w], acc, 0, 0, 0);
            }
            // acc = 16 * sum_d V q8 exactly (|acc| < 2^22): the 1/16 rides on
            // the column scale, a power of two, so qt is exact to the same bits
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if constexpr (TK4) {
                    const float2 w = vsf[pp][v >> 1];
                    c.qt[pp][v] = (float)acc[v] * ((v & 1) ? w.y : w.x) * qsjm[0];
                } else {
                    const float2 w = vsf[pp][v & 1];
                    c.qt[pp][v] = (float)acc[v] * ((v >> 1) ? w.y : w.x) * qsjm[(2 * pp + (v & 1)) % PPM];
                }
            }
        }
        {
            v4i accm = {0, 0, 0, 0};
#pragma unroll
            for (int w = 0; w < NWIN; ++w)
                accm = __builtin_amdgcn_mfma_i32_16x16x64_i8(Amu[w], mu[w], accm, 0, 0, 0);
            float4 md;                               // PIPE: lanes & 15 >= 8 store zeros into rows 8-15
            md.x = (float)accm[0] * qsl.x * musf;
            md.y = (float)accm[1] * qsl.y * musf;
            md.z = (float)accm[2] * qsl.z * musf;
            md.w = (float)accm[3] * qsl.w * musf;
            if (PIPE || (lane & 15) < 8)
                *reinterpret_cast<float4*>(mud + (lane & 15) * MUD_RS + 4 * kg) = md;
        }
        // the next unit's rows stream in under the previous unit's token
        // stage; issued after this unit's projection and centroid MFMAs
        // (measured against issuing it before them, right after the operand
        // reads: GLM 1M step 2.022 -> 2.005 ms, ragged batch 1.841 -> 1.822,
        // Llama unchanged; issuing it before the operand reads was slower
        // still)
        if (c.more) issue(c.nf, st_next);
        return c;
    };

    auto back = [&](const Carry& c, const float* mud) {
        flush_pend();                                // a unit not yet flushed by a front
        auto mud_at = [&](int page, int g) -> float { return mud[page * MUD_RS + g]; };
        const int p0 = c.p0, nvalid = c.nvalid;
        // ---- token reconstruction + PG-token LSE per (page, head) --------
        if constexpr (TK4) {
        // 4x4 block b = 4 kg + qd: page 4 gi + kg, tokens 4 qd .. 4 qd + 3 (A
        // lane 4 b + i: token 4 qd + i = r16), columns = heads (lane & 3).
        // One k step per basis column c; B = qt of the lane's own page, column
        // c (projection pair 2 gi + (c >> 2), element c & 3).  The token
        // scale rides on the coefficient operand (int8 x bf16 is exact in
        // fp32).  Lane (kg, qd, g) receives tokens 4 qd .. + 3 of (page, head g).
        auto tok4 = [&](int gi, int tb) -> v4f {
            const uint2 cw = c.c8w[gi][tb];
            const float cf = __uint_as_float(c.tw[gi][tb] << 16);
            v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t w = (k < 4) ? cw.x : cw.y;
                const float a = (float)(int8_t)(w >> (8 * (k & 3))) * cf;
                acc = __builtin_amdgcn_mfma_f32_4x4x1f32(a, c.qt[2 * gi + (k >> 2)][k & 3], acc, 0, 0, 0);
            }
            return acc;
        };
        const int qd = r16 >> 2;
        float ev[2] = {0.f, 0.f};
#pragma unroll
        for (int tb = 0; tb < NTB; ++tb) {
            const v4f x0 = tok4(0, tb), x1 = tok4(1, tb);
            ev[0] += __builtin_amdgcn_exp2f(x0[0]) + __builtin_amdgcn_exp2f(x0[1]) +
                     __builtin_amdgcn_exp2f(x0[2]) + __builtin_amdgcn_exp2f(x0[3]);
            ev[1] += __builtin_amdgcn_exp2f(x1[0]) + __builtin_amdgcn_exp2f(x1[1]) +
                     __builtin_amdgcn_exp2f(x1[2]) + __builtin_amdgcn_exp2f(x1[3]);
        }
        // sum over the 4 quads of a (page, head): lanes 4 apart in the row
#pragma unroll
        for (int gi = 0; gi < 2; ++gi) {
            ev[gi] += row_ror<4>(ev[gi]);
            ev[gi] += row_ror<8>(ev[gi]);
        }
        // quads 0-1 finish group 0, quads 2-3 group 1 (one log per lane)
        const int gsel = qd >> 1;
        const float tot = gsel ? ev[1] : ev[0];
        const int page = 4 * gsel + kg;
        const bool ok = (tot >= 0x1p-60f) && (tot <= 0x1p60f);
        float Sv;
        if (__builtin_expect(__ballot(!ok) == 0ull, 1)) {
            Sv = (mud_at(page, g_l) + __builtin_amdgcn_logf(tot)) * 0.6931471805599453f;
        } else {
            // exact-max form (rare)
            float Sa[2];
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                v4f x[NTB];
                float m = -INFINITY;
#pragma unroll
                for (int tb = 0; tb < NTB; ++tb) {
                    x[tb] = tok4(gi, tb);
                    m = fmaxf(m, fmaxf(fmaxf(x[tb][0], x[tb][1]), fmaxf(x[tb][2], x[tb][3])));
                }
                m = fmaxf(m, row_ror<4>(m));
                m = fmaxf(m, row_ror<8>(m));
                float f = 0.f;
#pragma unroll
                for (int tb = 0; tb < NTB; ++tb)
                    f += __builtin_amdgcn_exp2f(x[tb][0] - m) + __builtin_amdgcn_exp2f(x[tb][1] - m) +
                         __builtin_amdgcn_exp2f(x[tb][2] - m) + __builtin_amdgcn_exp2f(x[tb][3] - m);
                f += row_ror<4>(f);
                f += row_ror<8>(f);
                Sa[gi] = ((mud_at(4 * gi + kg, g_l) + m) + __builtin_amdgcn_logf(f)) * 0.6931471805599453f;
            }
            Sv = gsel ? Sa[1] : Sa[0];
        }
        const bool keep = (qd & 1) == 0 && page < nvalid && g_l < G;
        if (keep) {
            wrun = fmaxf(wrun, Sv);
            if constexpr (STG) sc_l[g_l * (c1 - c0 + 1) + (p0 - c0) + page] = Sv;
        }
        put_score(0, (((long)r * n_kv + h) * G + g_l) * (long)MP + p0 + page, Sv, keep);
        } else {
        // k-slot kg, step hh <-> basis column 2kg + hh (both operands);
        // tokens in blocks of 16 (tb < PG / 16)
        auto tok_group = [&](int gi, int tb) -> v4f {   // cs * (C8 qt) of group gi, 4 tokens
            v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ps = 0; ps < PPM; ++ps) {
                const int page = gi * PPM + ps;
                const uint32_t w = c.tw[page][tb];
                // the token scale rides on the coefficient operand: int8 x
                // bf16 is exact in fp32
                const float cf = __uint_as_float(w & 0xFFFF0000u);
                const float a0 = (float)(int8_t)w * cf, a1 = (float)(int8_t)(w >> 8) * cf;
                // qt is already zero where this lane's column is not page slot ps
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, c.qt[page >> 1][page & 1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, c.qt[page >> 1][2 + (page & 1)], acc, 0, 0, 0);
            }
            return acc;
        };
        // 16-token LSE taken relative to the centroid term: tok - mud =
        // cs * acc.  The exp2 sum is exact whenever it lies in [2^-60, 2^60]
        // (no overflow; flushed terms < 2^-62 of the sum).  All groups are
        // formed first (independent matrix-core chains interleave), then one
        // wave-wide test picks this fast form or the exact-max recomputation.
        // Per-lane partial sums (4 tokens) of every group, then one
        // transposing reduction per 4 groups: two row-pair swaps and one
        // half swap leave group 4s + kg's 16-token total in row kg (same
        // pairing and order as a per-group butterfly, so the same bits).
        // Each lane then finishes only its own row's group.
        constexpr int NSET = (NGRP + 3) / 4;
        float ev[NGRP];
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
            ev[gi] = 0.f;
#pragma unroll
            for (int tb = 0; tb < NTB; ++tb) {
                const v4f x = tok_group(gi, tb);
                ev[gi] += __builtin_amdgcn_exp2f(x[0]) + __builtin_amdgcn_exp2f(x[1]) +
                          __builtin_amdgcn_exp2f(x[2]) + __builtin_amdgcn_exp2f(x[3]);
            }
        }
        float tot[NSET];
#pragma unroll
        for (int sx = 0; sx < NSET; ++sx) {
            auto pair16 = [](float u, float v) {
                const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(u), __float_as_uint(v), false, false);
                return __uint_as_float(r[0]) + __uint_as_float(r[1]);
            };
            if constexpr (NGRP >= 4) {
                const float A = pair16(ev[4 * sx], ev[4 * sx + 1]);      // rows: g0 01, g1 01, g0 23, g1 23
                const float B = pair16(ev[4 * sx + 2], ev[4 * sx + 3]);  // rows: g2 01, g3 01, g2 23, g3 23
                const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(A), __float_as_uint(B), false, false);
                tot[sx] = __uint_as_float(r[0]) + __uint_as_float(r[1]); // row k: group 4 sx + k
            } else {
                tot[sx] = xor32_sum(pair16(ev[0], ev[1]));               // row k: group k & 1
            }
        }
        auto grp_of = [&](int sx) { return (NGRP >= 4) ? 4 * sx + kg : (kg & 1); };
        bool ok = true;
#pragma unroll
        for (int sx = 0; sx < NSET; ++sx) ok = ok && (tot[sx] >= 0x1p-60f) && (tot[sx] <= 0x1p60f);
        float Sv[NSET];
        if (__builtin_expect(__ballot(!ok) == 0ull, 1)) {
#pragma unroll
            for (int sx = 0; sx < NSET; ++sx)
                Sv[sx] = (mud_at(grp_of(sx) * PPM + psub_l, g_l) + __builtin_amdgcn_logf(tot[sx])) *
                         0.6931471805599453f;
        } else {
            // exact-max form (rare): every lane computes every group
            float Sa[NGRP];
#pragma unroll
            for (int gi = 0; gi < NGRP; ++gi) {
                v4f x[NTB];
                float m = -INFINITY;
#pragma unroll
                for (int tb = 0; tb < NTB; ++tb) {
                    x[tb] = tok_group(gi, tb);
                    m = fmaxf(m, fmaxf(fmaxf(x[tb][0], x[tb][1]), fmaxf(x[tb][2], x[tb][3])));
                }
                m = xor32_max(xor16_max(m));
                float f = 0.f;
#pragma unroll
                for (int tb = 0; tb < NTB; ++tb)
                    f += __builtin_amdgcn_exp2f(x[tb][0] - m) + __builtin_amdgcn_exp2f(x[tb][1] - m) +
                         __builtin_amdgcn_exp2f(x[tb][2] - m) + __builtin_amdgcn_exp2f(x[tb][3] - m);
                f = xor32_sum(xor16_sum(f));
                Sa[gi] = ((mud_at(gi * PPM + psub_l, g_l) + m) + __builtin_amdgcn_logf(f)) * 0.6931471805599453f;
            }
#pragma unroll
            for (int sx = 0; sx < NSET; ++sx) {
                float v = Sa[0];
#pragma unroll
                for (int gi = 1; gi < NGRP; ++gi) v = (grp_of(sx) == gi) ? Sa[gi] : v;
                Sv[sx] = v;
            }
        }
        float tmax = -INFINITY;
        const bool row_owner = (NGRP >= 4) || (kg < 2);      // rows 2, 3 repeat rows 0, 1
#pragma unroll
        for (int sx = 0; sx < NSET; ++sx) {
            const int page = grp_of(sx) * PPM + psub_l;
            const bool keep = row_owner && (page < nvalid) && (g_l < G);
            if (keep) {
                tmax = fmaxf(tmax, Sv[sx]);
                if constexpr (STG) sc_l[g_l * (c1 - c0 + 1) + (p0 - c0) + page] = Sv[sx];
            }
            put_score(STG ? 0 : sx, (((long)r * n_kv + h) * G + g_l) * (long)MP + p0 + page, Sv[sx], keep);
        }
        wrun = fmaxf(wrun, tmax);
        }
    };
    // a pending DMA's source registers stay allocated until the unit after
    // it has been waited for (a write to one would have to wait for the DMA)
    auto pin = [&](const Carry& c) {
        if (c.more) {
#pragma unroll
            for (int i = 0; i < (PK ? NDI : 1); ++i) asm volatile("" :: "v"(c.nf.off[i]));
#pragma unroll
            for (int i = 0; i < (PK ? 1 : NDI); ++i) asm volatile("" :: "v"(c.nf.addr[i]));
            asm volatile("" :: "v"(c.nf.mus));
        }
    };
    if constexpr (!PIPE) {
        for (int u = wave; u < n_units; u += 2 * SC_WAVES) {
            float* ma = reinterpret_cast<float*>(sa_l[wave]);
            float* mb = reinterpret_cast<float*>(sb_l[wave]);
            Carry c = front(u, sa_l[wave], sb_l[wave], ma);
            wave_lds_sync();
            back(c, ma);
            pin(c);
            wave_lds_sync();                           // stages reused by the unit after next
            if (u + SC_WAVES < n_units) {
                c = front(u + SC_WAVES, sb_l[wave], sa_l[wave], mb);
                wave_lds_sync();
                back(c, mb);
                pin(c);
                wave_lds_sync();
            }
        }
    } else if (wave < n_units) {
        int u = wave;
        Carry ca = front(u, sa_l[wave], sb_l[wave], mud_l[wave][0]);
        for (;;) {
            u += SC_WAVES;
            if (u >= n_units) { wave_lds_sync(); back(ca, mud_l[wave][0]); break; }
            Carry cb = front(u, sb_l[wave], sa_l[wave], mud_l[wave][1]);
            back(ca, mud_l[wave][0]);
            pin(ca);
            u += SC_WAVES;
            if (u >= n_units) { wave_lds_sync(); back(cb, mud_l[wave][1]); break; }
            ca = front(u, sa_l[wave], sb_l[wave], mud_l[wave][0]);
            back(cb, mud_l[wave][1]);
            pin(cb);
        }
    }
    flush_pend();
    // per-head maxima of the workgroup -> LDS (ordered-uint atomic max), one
    // atomic per head column per row
#pragma unroll
    for (int o = GW; o < 16; o <<= 1)        // max over the lanes of one head column
        wrun = fmaxf(wrun, o == 4 ? row_ror<4>(wrun) : o == 8 ? row_ror<8>(wrun) : row_ror<2>(wrun));
    if ((TK4 || NGRP >= 4 || kg < 2) && (lane & 15) < GW && (lane & 15) < G) atomicMax(&wmax[lane & 15], f2u(wrun));
    __syncthreads();
    if constexpr (STG) {
        const int n = c1 - c0;
        float* srow = score_h + ((long)r * n_kv + h) * G * (long)MP + c0;
        for (int g = 0; g < G; ++g)
            for (int p = tid; p < n; p += SC_BLOCK) srow[(long)g * MP + p] = sc_l[g * (n + 1) + p];
    }
    if (tid < 16) pm_out[(long)tid * Z] = u2f(wmax[tid]);
}

}  // namespace locks

using namespace locks;

extern "C" int32_t locks_score_auto_chunk(int32_t n_req, int32_t n_kv, int32_t max_pages) {
    // ~512 workgroups (2 per CU on a 256-CU MI355X) over all (request, kv
    // head, 8-page tile) units; a workgroup scores whole tiles of one kv head.
    // With several requests the grid is sized for max_pages per row, and the
    // shorter rows of a ragged batch leave their tail chunks idle, so aim at
    // ~1024 (GLM batch {256K,192K,128K,64K}: 27.9 -> 23.5 us per launch).
    const long tiles = (long)cdiv(max_pages > 0 ? max_pages : 1, SC_TILE);
    const long units = tiles * (n_kv > 0 ? n_kv : 1) * (n_req > 0 ? n_req : 1);
    const long target = n_req > 1 ? 1024 : 512;
    long ct = (units + target - 1) / target;             // tiles per workgroup (one kv head)
    // Small grids: at least units / 256 tiles per workgroup, up to 4 (one
    // unit per wave): GLM G = 16 step at 32K 0.996 (2 tiles) vs 1.005 ms (1),
    // 64K 1.032 (4) vs 1.056 (2), 128K 1.219 (4) vs 1.242 (8) vs 1.410 (2);
    // at 16K, 256 units, the floor is 1 (32 workgroups measured 1.284
    // against 1.215 ms)
    const long floor_ct = units / 256 < 4 ? units / 256 : 4;
    if (ct < floor_ct) ct = floor_ct;
    if (ct < 1) ct = 1;
    if (ct > SC_MAX_CHUNK / SC_TILE) ct = SC_MAX_CHUNK / SC_TILE;
    return (int32_t)(ct * SC_TILE);
}

extern "C" int32_t locks_score_num_chunks(int32_t max_pages, int32_t chunk) {
    if (chunk <= 0) return -1;
    return cdiv(max_pages > 0 ? max_pages : 1, chunk);
}

extern "C" int32_t locks_score_rki4(
    const uint16_t* q, int64_t q_stride_req, int64_t q_stride_head,
    const uint8_t* v4, const uint16_t* vs, const int8_t* c8, const uint16_t* cs,
    const int8_t* mu8, const uint16_t* mus, const int64_t* slab_row_bytes, int32_t num_blocks,
    const int32_t* block_table, int64_t bt_stride, int32_t bt_cols,
    const int32_t* n_sel_hi, float* score_h, int32_t max_pages,
    float* page_max, int32_t chunk,
    int32_t n_req, int32_t n_kv, int32_t G, int32_t head_dim, int32_t page,
    float sm_scale, void* stream)
{
    LOCKS_REQUIRE((head_dim == 64 || head_dim == 128 || head_dim == 256) && (page == 16 || page == 32 || page == 64),
                  "locks_score_rki4: head_dim %d / page %d outside {64,128,256} x {16,32,64}", head_dim, page);
    LOCKS_REQUIRE(G >= 1 && G <= 16, "locks_score_rki4: G=%d outside [1, 16]", G);
    LOCKS_REQUIRE(n_req >= 0 && n_req <= 65535 && n_kv >= 1 && n_kv <= 65535,
                  "locks_score_rki4: n_req=%d / n_kv=%d outside the grid limits", n_req, n_kv);
    LOCKS_REQUIRE(q_stride_head % 8 == 0 && q_stride_req % 8 == 0,
                  "locks_score_rki4: q strides must be multiples of 8 elements (16-byte loads)");
    const SlabRows S = slab_rows(v4, vs, c8, cs, mu8, mus, slab_row_bytes, head_dim, page);
    LOCKS_REQUIRE(slab_rows_ok(S, head_dim, page),
                  "locks_score_rki4: slab row strides below the field sizes or misaligned");
    LOCKS_REQUIRE(slab_rows_extent(S, (long)num_blocks * n_kv) < (1L << 32),
                  "locks_score_rki4: slab too large for 32-bit offsets");
    LOCKS_REQUIRE(num_blocks >= 1 && bt_cols >= 1 && max_pages >= 1,
                  "locks_score_rki4: empty geometry (num_blocks=%d bt_cols=%d max_pages=%d)",
                  num_blocks, bt_cols, max_pages);
    LOCKS_REQUIRE(chunk >= SC_TILE && chunk % SC_TILE == 0 && chunk <= SC_MAX_CHUNK,
                  "locks_score_rki4: chunk %d must be a multiple of %d in [%d, %d]", chunk, SC_TILE,
                  SC_TILE, SC_MAX_CHUNK);
    LOCKS_REQUIRE(q && v4 && vs && c8 && cs && mu8 && mus && block_table && n_sel_hi && score_h && page_max,
                  "locks_score_rki4: null pointer argument");
    if (n_req == 0) return 0;
    const int Z = cdiv(max_pages, chunk);
    dim3 grid(Z, n_kv, n_req);
    const size_t dyn = (size_t)chunk * sizeof(int);
    // one request and a wide group: the scores are staged in LDS when the
    // chunk's fit (GLM 1M, G = 16: step 2.051 -> 2.017 ms; at Llama's G = 4
    // a unit stores 32 scores, and the closing copy cost more than it saved:
    // 1.035 -> 1.052 ms)
    const bool stg = G > 8 && (long)chunk * G <= SC_STAGE_F;
    hipStream_t st = (hipStream_t)stream;
    // packed rows: all six fields of a row together, in the kernel's order,
    // rows of one common stride (any stride >= the fields: the reference's
    // AoS record rounds to 64 B)
    const long RSB = S.sv4;
    const bool packed = RSB >= 5L * head_dim + 10L * page + 18 && S.svs == RSB && S.sc8 == RSB &&
                        S.scs == RSB && S.smu == RSB && S.smus == RSB &&
                        S.mu == S.v4 + 4L * head_dim && S.c8 == S.mu + head_dim &&
                        S.cs == S.c8 + 8L * page && S.vs == S.cs + 2L * page && S.mus == S.vs + 16;
#define LAUNCH_P(GWV, DV, PGV, PKV, PIPEV, STGV)                                               \
    hipLaunchKernelGGL((rki4_score_kernel<GWV, DV, PGV, PKV, PIPEV, STGV>), grid, dim3(SC_BLOCK), dyn, st, q, \
                       (long)q_stride_req, (long)q_stride_head, S,                             \
                       num_blocks, block_table, (long)bt_stride, bt_cols, n_sel_hi,            \
                       score_h, max_pages, page_max, n_kv, G, sm_scale, chunk)
    // one request: ~512 workgroups, two per CU, each wave pipelining its
    // units; several requests: the ~1024-workgroup grid of the auto chunk
    // fits three per CU only without the pipeline's registers and buffer
    // (ragged GLM batch step 2.05 -> 1.95 ms)
#define LAUNCH(GWV, DV, PGV, PKV)                                    \
    do {                                                             \
        if (n_req == 1 && stg) LAUNCH_P(GWV, DV, PGV, PKV, true, (GWV == 16)); \
        else if (n_req == 1) LAUNCH_P(GWV, DV, PGV, PKV, true, false); \
        else LAUNCH_P(GWV, DV, PGV, PKV, false, false);              \
    } while (0)
#define LAUNCH_GP(DV, PGV, PKV)                    \
    do {                                           \
        if (G <= 4) LAUNCH(4, DV, PGV, PKV);       \
        else if (G <= 8) LAUNCH(8, DV, PGV, PKV);  \
        else LAUNCH(16, DV, PGV, PKV);             \
    } while (0)
#define LAUNCH_G(DV, PGV)                          \
    do {                                           \
        if (packed) LAUNCH_GP(DV, PGV, true);      \
        else LAUNCH_GP(DV, PGV, false);            \
    } while (0)
    if (page == 16) {
        if (head_dim == 128) LAUNCH_G(128, 16);
        else if (head_dim == 64) LAUNCH_G(64, 16);
        else LAUNCH_G(256, 16);
    } else if (page == 32) {
        if (head_dim == 128) LAUNCH_G(128, 32);
        else if (head_dim == 64) LAUNCH_G(64, 32);
        else LAUNCH_G(256, 32);
    } else {
        if (head_dim == 128) LAUNCH_G(128, 64);
        else if (head_dim == 64) LAUNCH_G(64, 64);
        else LAUNCH_G(256, 64);
    }
#undef LAUNCH_G
#undef LAUNCH_GP
#undef LAUNCH
#undef LAUNCH_P
    return check_launch("rki4_score_kernel");
}
