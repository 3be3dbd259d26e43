// rki4 summary build for gfx950: finalized K pages -> six-slab summaries.
//
// Op sequence of the reference builder (selection/rki4_build.py:147-158
// _write_pre, :93-129 eigh, :178-225 _write_post, :161-175 int4 pack), per
// (block, kv head):
//   mu = mean_t K; dc = K - mu; Gm = dc dc^T (16 x 16)
//   S2, U = eigh(Gm) ascending; S8 = sqrt(max(S2[-8:], 1e-10)); U8 = U[:, -8:]
//   C = U8 * S8 ; V = dc^T U8 / S8
//   vs = max(|V|_d / 7, 1e-8);  Vq = clamp(rint(V / vs), -8, 7)  -> int4 packed
//   cs = max(|C|_r / 127, 1e-8); Cq = clamp(rint(C / cs), +-127)
//   ms = max(|mu| / 127, 1e-8); muq = clamp(rint(mu / ms), +-127)
//   scales stored bf16 (RNE); tag = K[15, kh, 0:8].
//
// MI355X mapping: one wave per (block, kv head).  The page is staged in LDS
// as fp32; the gram runs on v_mfma_f32_16x16x4_f32 (A and B operands are the
// same lane values because Gm = dc dc^T); the eigendecomposition is a
// parallel cyclic Jacobi (round-robin ordering: 8 disjoint rotations per
// step, 15 steps per sweep) on the 16x16 matrix in LDS -- the reference
// calls a batched LAPACK/cuSOLVER eigh; any eigensolver agrees with it only
// up to eigenvector sign/rotation, which the summary tolerates by design.
// The quantize/pack stage is shared with locks_pack_rki4, which takes the
// eigenpairs from the caller and is bit-exact to the reference op order
// (V accumulated over t in ascending order with separately rounded multiply
// and add, IEEE division, round-half-even).
#include <algorithm>

#include "locks_common.h"
#include "locks_hip.h"

namespace locks {

constexpr int BD_RNK = 8;
// build grid cap (waves stride over the rest): a few resident rounds on 256 CUs
constexpr long BD_MAX_GRID = 4096;

// Per-wave LDS image of one (block, kv head) page of PG tokens x D dims.
template <int D, int PG>
struct WaveLds {
    float dc[PG][D + 1];         // centred page (padded rows)
    float mu[D];
    float A[PG][PG + 1];         // gram, rotated in place
    float U[PG][PG + 1];         // accumulated eigenvectors (columns)
    // second buffers of the page-64 Jacobi step (one element per row 1 x 1
    // otherwise)
    float A2[PG == 64 ? PG : 1][PG + 1];
    float U2[PG == 64 ? PG : 1][PG + 1];
    float cc[PG], ss[PG];
    float S8[BD_RNK];
    int col[BD_RNK];             // eigen column of basis r (ascending top-8)
    float red[BD_RNK][kWave / 8];
};
// waves per workgroup: as many page images as fit 160 KB of LDS, at most 4;
// d = 512 (the MLA latent, ~37 KB per image) runs one
template <int D, int PG> constexpr int bd_waves() {
    if (D >= 512) return 1;
    constexpr int n = (160 * 1024) / (int)sizeof(WaveLds<D, PG>);
    return n >= 4 ? 4 : n;
}

// quantize + pack one page from mu (LDS), dc (LDS), U8 = U[:, col[r]],
// S8 (LDS), writing the six slab rows.  Lane l owns the packed bytes
// j = l + 64 k (d = 2j, 2j + 1).
template <int D, int PG>
__device__ __forceinline__ void pack_page(WaveLds<D, PG>& L, long row, const SlabRows& S) {
    constexpr int NK = (D / 2 + 63) / 64;      // packed bytes per lane (d = 64: lanes < 32)
    const int lane = threadIdx.x & 63;
    auto own = [&](int k) { return lane + 64 * k < D / 2; };
    // V[d][r]: sequential over t, separately rounded
    float V[NK][2][BD_RNK];
#pragma unroll
    for (int k = 0; k < NK; ++k)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int d = 2 * (lane + 64 * k) + e;
#pragma unroll
            for (int r = 0; r < BD_RNK; ++r) {
                // d <= 256: a compiler barrier keeps one column's operands
                // live at a time (hoisting all 16 x 8 basis values costs ~130
                // VGPRs and halves the occupancy).  d = 512 runs one wave per
                // SIMD anyway (its LDS image), so there the hoisting is free
                // and the barrier would only multiply the LDS reloads.
                if constexpr (D <= 256) asm volatile("" ::: "memory");
                float acc = 0.f;
                const int c = L.col[r];
                if (own(k))
                    for (int t = 0; t < PG; ++t) acc = __fadd_rn(acc, __fmul_rn(L.dc[t][d], L.U[t][c]));
                V[k][e][r] = __fdiv_rn(acc, L.S8[r]);
            }
        }
    // per-column absmax over d
    float vsc[BD_RNK];
#pragma unroll
    for (int r = 0; r < BD_RNK; ++r) {
        float am = 0.f;
#pragma unroll
        for (int k = 0; k < NK; ++k) am = fmaxf(am, fmaxf(fabsf(V[k][0][r]), fabsf(V[k][1][r])));
        am = wave_max(am);
        vsc[r] = fmaxf(__fdiv_rn(am, 7.f), 1e-8f);
    }
    uint8_t* vrow = S.v4 + row * S.sv4;
#pragma unroll
    for (int r = 0; r < BD_RNK; ++r)
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int lo = (int)fminf(fmaxf(rintf(__fdiv_rn(V[k][0][r], vsc[r])), -8.f), 7.f);
            const int hi = (int)fminf(fmaxf(rintf(__fdiv_rn(V[k][1][r], vsc[r])), -8.f), 7.f);
            if (own(k)) vrow[r * (D / 2) + lane + 64 * k] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
        }
    if (lane < BD_RNK) reinterpret_cast<uint16_t*>(S.vs + row * S.svs)[lane] = f32_to_bf16(vsc[lane]);
    // coefficients: lane t < PG owns token t
    if (lane < PG) {
        const int t = lane;
        float C[BD_RNK];
        float am = 0.f;
#pragma unroll
        for (int r = 0; r < BD_RNK; ++r) {
            C[r] = __fmul_rn(L.U[t][L.col[r]], L.S8[r]);
            am = fmaxf(am, fabsf(C[r]));
        }
        const float csc = fmaxf(__fdiv_rn(am, 127.f), 1e-8f);
        int8_t* crow = reinterpret_cast<int8_t*>(S.c8 + row * S.sc8) + t * BD_RNK;
#pragma unroll
        for (int r = 0; r < BD_RNK; ++r)
            crow[r] = (int8_t)fminf(fmaxf(rintf(__fdiv_rn(C[r], csc)), -127.f), 127.f);
        reinterpret_cast<uint16_t*>(S.cs + row * S.scs)[t] = f32_to_bf16(csc);
    }
    // centroid
    float am = 0.f;
#pragma unroll
    for (int k = 0; k < NK; ++k)
        if (own(k)) am = fmaxf(am, fmaxf(fabsf(L.mu[2 * (lane + 64 * k)]), fabsf(L.mu[2 * (lane + 64 * k) + 1])));
    am = wave_max(am);
    const float msc = fmaxf(__fdiv_rn(am, 127.f), 1e-8f);
#pragma unroll
    for (int k = 0; k < NK; ++k)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int d = 2 * (lane + 64 * k) + e;
            if (own(k)) reinterpret_cast<int8_t*>(S.mu + row * S.smu)[d] = (int8_t)fminf(fmaxf(rintf(__fdiv_rn(L.mu[d], msc)), -127.f), 127.f);
        }
    if (lane == 0) *reinterpret_cast<uint16_t*>(S.mus + row * S.smus) = f32_to_bf16(msc);
}

// Parallel cyclic Jacobi on L.A (N x N symmetric, N = page = 16, 32 or 64);
// eigenvectors -> L.U columns.  Round-robin pairing of step `step`: index 0
// stays, 1..N-1 rotate; the pair of position k (1 <= k < N/2) is
// (at(k), at(N-1-k)), position 0 pairs index 0 with at(0), where
// at(k) = 1 + (k + step) % (N - 1).
template <int N>
__device__ __forceinline__ int rr_at(int k, int step) { return 1 + (k + step) % (N - 1); }
template <int N>
__device__ __forceinline__ int rr_partner(int i, int step) {
    if (i == 0) return rr_at<N>(0, step);
    const int k = (i - 1 - step + (N - 1)) % (N - 1);
    return k == 0 ? 0 : rr_at<N>(N - 1 - k, step);
}

// Parallel cyclic Jacobi on the N x N symmetric matrix in L.A (eigenvalues
// end on the diagonal, eigenvectors in the columns of L.U).  One step applies
// the N/2 disjoint rotations of the round-robin schedule as one two-sided
// update A'' = J^T A J read entirely from the old A:
//   A''[i][j] = c_j (c_i A[i][j] + s_i A[pi][j]) + s_j (c_i A[i][pj] + s_i A[pi][pj])
//   U'[i][j]  = c_j U[i][j] + s_j U[i][pj]
// Lane l owns column j = l % N of rows l / N + (64 / N) e.  A wave executes
// its LDS instructions in order, so the old values every lane reads are read
// before any lane writes (the asm barriers keep the compiler from moving the
// accesses across each other): two dependent LDS round trips per step.
// Rotation parameters use the hardware reciprocal and reciprocal square root
// (~1 ulp): a rotation only has to reduce the off-diagonal mass, and the
// result is checked through the quantised summary, not bit for bit.
template <int N, class W>
__device__ void jacobi(W& L) {
    static_assert(N == 16 || N == 32 || N == 64, "page 16, 32 or 64");
    constexpr int RS = kWave / N, RPL = N * N / kWave;   // row stride, rows per lane
    constexpr int SWEEPS = N == 16 ? 12 : N == 32 ? 16 : 20;
    const int lane = threadIdx.x & 63;
    const int j = lane % N, r0 = lane / N;
    for (int i = lane; i < N * N; i += kWave) L.U[i / N][i % N] = (i / N == i % N) ? 1.f : 0.f;
    wave_lds_sync();
    for (int sweep = 0; sweep < SWEEPS; ++sweep) {
        // convergence test: off-diagonal mass vs diagonal
        float off = 0.f, dia = 0.f;
        for (int i = lane; i < N * N; i += kWave) {
            const float a = L.A[i / N][i % N];
            if (i / N == i % N) dia += a * a; else off += a * a;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            off += __shfl_xor(off, o, kWave);
            dia += __shfl_xor(dia, o, kWave);
        }
        // wave-uniform (also exits on 0/0).  fp32 rounding leaves off/dia
        // near 1e-14 (asymmetric residues of order eps * |lambda|), so the
        // bound sits above that floor: 5-6 sweeps at N = 16 instead of
        // running out the sweep limit, with the same top-8 eigenvalue
        // accuracy (~3e-6 rel).
        if (!(off > 1e-12f * dia)) break;
        for (int step = 0; step < N - 1; ++step) {
            // page 64: A / U alternate between the two buffers step by step
            float (*Ac)[N + 1] = (N == 64 && (step & 1)) ? L.A2 : L.A;
            if (lane < N / 2) {
                const int p = lane == 0 ? 0 : rr_at<N>(lane, step);
                const int q = lane == 0 ? rr_at<N>(0, step) : rr_at<N>(N - 1 - lane, step);
                const float apq = Ac[p][q], app = Ac[p][p], aqq = Ac[q][q];
                float c = 1.f, sn = 0.f;
                if (fabsf(apq) > 1e-30f) {                 // smaller: nothing to rotate away
                    const float theta = (aqq - app) * __builtin_amdgcn_rcpf(2.f * apq);
                    const float t = copysignf(__builtin_amdgcn_rcpf(fabsf(theta) +
                                                                    __builtin_amdgcn_sqrtf(theta * theta + 1.f)),
                                              theta);
                    c = __builtin_amdgcn_rsqf(t * t + 1.f);
                    sn = t * c;
                }
                L.cc[p] = c; L.ss[p] = -sn;
                L.cc[q] = c; L.ss[q] = sn;
            }
            asm volatile("" ::: "memory");
            const int pj = rr_partner<N>(j, step);
            const float cj = L.cc[j], sj = L.ss[j];
            if constexpr (N == 64) {
                // 64 rows per lane: read the current buffers, write the
                // other ones (the old values are never overwritten inside the
                // step, so nothing has to be held in registers), then swap
                float (*Uc)[N + 1] = (step & 1) ? L.U2 : L.U;
                float (*An)[N + 1] = (step & 1) ? L.A : L.A2;
                float (*Un)[N + 1] = (step & 1) ? L.U : L.U2;
                for (int i = 0; i < N; ++i) {
                    const int pi = rr_partner<N>(i, step);
                    const float ci = L.cc[i], si = L.ss[i];
                    An[i][j] = cj * (ci * Ac[i][j] + si * Ac[pi][j]) + sj * (ci * Ac[i][pj] + si * Ac[pi][pj]);
                    Un[i][j] = cj * Uc[i][j] + sj * Uc[i][pj];
                }
                asm volatile("" ::: "memory");
                continue;
            }
            float na[RPL], nu[RPL];
#pragma unroll
            for (int e = 0; e < RPL; ++e) {
                const int i = r0 + RS * e, pi = rr_partner<N>(i, step);
                const float ci = L.cc[i], si = L.ss[i];
                na[e] = cj * (ci * L.A[i][j] + si * L.A[pi][j]) + sj * (ci * L.A[i][pj] + si * L.A[pi][pj]);
                nu[e] = cj * L.U[i][j] + sj * L.U[i][pj];
            }
            asm volatile("" ::: "memory");
#pragma unroll
            for (int e = 0; e < RPL; ++e) {
                L.A[r0 + RS * e][j] = na[e];
                L.U[r0 + RS * e][j] = nu[e];
            }
            asm volatile("" ::: "memory");
        }
        if constexpr (N == 64) {
            // a sweep has 63 steps: the result sits in the second buffers
            for (int i = 0; i < N; ++i) {
                L.A[i][lane] = L.A2[i][lane];
                L.U[i][lane] = L.U2[i][lane];
            }
            asm volatile("" ::: "memory");
        }
    }
}

// eigenvalues on the diagonal of L.A -> ascending ranks -> top-8 columns
template <int N, class W>
__device__ void select_top8(W& L) {
    const int lane = threadIdx.x & 63;
    if (lane < N) {
        const float li = L.A[lane][lane];
        int rank = 0;
        for (int j = 0; j < N; ++j) {
            const float lj = L.A[j][j];
            rank += (lj < li) || (lj == li && j < lane);
        }
        if (rank >= N - BD_RNK) {
            const int r = rank - (N - BD_RNK);
            L.col[r] = lane;
            L.S8[r] = __fsqrt_rn(fmaxf(li, 1e-10f));
        }
    }
    wave_lds_sync();
}

// Grid: capped, waves stride over (layer, block, kv head).  Layer l reads K from
// k_layers[l] (or kc for a single-layer call) and writes slab rows offset by
// l * layer_rows.  n_dev, when given, is a device count of valid entries of
// `blocks` (at most n_blocks): the refresh producers size the grid to the
// host-known bound and the list is compacted on the device.
template <int D, int PG = 16>
__global__ __launch_bounds__((bd_waves<D, PG>() * kWave)) void rki4_build_kernel(
    const uint16_t* __restrict__ kc, const uint64_t* __restrict__ k_layers,
    long k_sb, long k_st, long k_sh, int NB,
    const int* __restrict__ blocks, const int* __restrict__ n_dev, int n_blocks, int n_kv,
    int n_layers, long layer_rows, SlabRows S, uint16_t* __restrict__ tag)
{
    constexpr int NW = bd_waves<D, PG>();
    __shared__ WaveLds<D, PG> lds[NW];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    WaveLds<D, PG>& L = lds[wave];
    const int nb_valid = n_dev ? min(*n_dev, n_blocks) : n_blocks;
    const long per_layer = (long)nb_valid * n_kv;
    // one wave per (layer, block index, kv head), grid-stride
    for (long item = (long)blockIdx.x * NW + wave; item < per_layer * n_layers;
         item += (long)gridDim.x * NW) {
        const int layer = (int)(item / per_layer);
        const long rem = item - (long)layer * per_layer;
        const int bi = (int)(rem / n_kv), kh = (int)(rem % n_kv);
        const int blk = blocks[bi];
        if (blk < 0 || blk >= NB) continue;                        // masked (profile pass)
        const long row = (long)layer * layer_rows + (long)blk * n_kv + kh;
        const uint16_t* kbase = k_layers ? reinterpret_cast<const uint16_t*>(k_layers[layer]) : kc;
        const uint16_t* kp = kbase + (long)blk * k_sb + (long)kh * k_sh;

        // stage K (fp32) and the centroid (sequential sum over t, then / PG)
        for (int i = lane; i < PG * D / 8; i += kWave) {
            const int t = i / (D / 8), d0 = (i % (D / 8)) * 8;
            const uint4 w = *reinterpret_cast<const uint4*>(kp + (long)t * k_st + d0);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                L.dc[t][d0 + 2 * e] = bf16lo(ws[e]);
                L.dc[t][d0 + 2 * e + 1] = bf16hi(ws[e]);
            }
        }
        if (lane < 8) tag[row * 8 + lane] = kp[(long)(PG - 1) * k_st + lane];
        wave_lds_sync();
        for (int d = lane; d < D; d += kWave) {
            float acc = 0.f;
            for (int t = 0; t < PG; ++t) acc = __fadd_rn(acc, L.dc[t][d]);
            const float m = __fdiv_rn(acc, (float)PG);
            L.mu[d] = m;
            for (int t = 0; t < PG; ++t) L.dc[t][d] = __fsub_rn(L.dc[t][d], m);
        }
        wave_lds_sync();

        // gram on the matrix core: Gm[i][j] = sum_d dc[i][d] dc[j][d], in
        // 16 x 16 blocks (bi, bj) of the PG x PG matrix
        {
            const int i = lane & 15, kq = lane >> 4;
#pragma unroll 1
            for (int bi = 0; bi < PG / 16; ++bi)
#pragma unroll
                for (int bj = 0; bj < PG / 16; ++bj) {
                    v4f g = {0.f, 0.f, 0.f, 0.f};
                    for (int s = 0; s < D / 4; ++s) {
                        const float a = L.dc[16 * bi + i][4 * s + kq];
                        const float b = L.dc[16 * bj + i][4 * s + kq];
                        g = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, g, 0, 0, 0);
                    }
#pragma unroll
                    for (int v = 0; v < 4; ++v) L.A[16 * bi + 4 * kq + v][16 * bj + i] = g[v];
                }
        }
        wave_lds_sync();
        jacobi<PG>(L);
        select_top8<PG>(L);
        pack_page<D, PG>(L, row, S);
    }
}

// locks_pack_rki4: quantize + pack given the caller's eigen decomposition.
__global__ __launch_bounds__(4 * kWave) void rki4_pack_kernel(
    const float* __restrict__ mu, const float* __restrict__ dc, const float* __restrict__ S2,
    const float* __restrict__ U, const int* __restrict__ rows, int n, SlabRows S)
{
    constexpr int BD_D = 128, BD_PG = 16;
    __shared__ WaveLds<BD_D, BD_PG> lds[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    WaveLds<BD_D, BD_PG>& L = lds[wave];
    const long item = (long)blockIdx.x * 4 + wave;
    if (item >= n) return;
    for (int i = lane; i < BD_PG * BD_D; i += kWave) L.dc[i / BD_D][i % BD_D] = dc[item * BD_PG * BD_D + i];
    for (int i = lane; i < BD_D; i += kWave) L.mu[i] = mu[item * BD_D + i];
    for (int i = lane; i < BD_PG * BD_PG; i += kWave) L.U[i / BD_PG][i % BD_PG] = U[item * BD_PG * BD_PG + i];
    if (lane < BD_RNK) {
        const int c = BD_PG - BD_RNK + lane;                 // ascending input: top 8 = last 8
        L.col[lane] = c;
        L.S8[lane] = __fsqrt_rn(fmaxf(S2[item * BD_PG + c], 1e-10f));
    }
    wave_lds_sync();
    pack_page<BD_D, BD_PG>(L, rows[item], S);
}

// ---- refresh lifecycle: which blocks to (re)build --------------------------
// Reference producers: selection/build.py:372-384 _tail_blocks, :415-427
// _bulk_blocks, :472-488 _delta_select (rki4_build.py:264-315 call them).
// One thread per candidate page marks its physical block in a byte map
// (duplicates collapse: pages shared by several requests are built once);
// refresh_compact_kernel turns the map into a list plus a device count and
// clears the map again.  No host sync on any mode.
constexpr int RF_THREADS = 256;

__device__ __forceinline__ bool tags_differ(uint4 a, uint4 b) {
    // bf16 values compared as numbers, like the reference's float compare:
    // NaN (the never-built tag) differs from everything, -0 equals +0
    const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
    bool d = false;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        d |= (bf16lo(wa[e]) != bf16lo(wb[e])) | (bf16hi(wa[e]) != bf16hi(wb[e]));
    return d;
}

__global__ __launch_bounds__(RF_THREADS) void refresh_mark_kernel(
    int mode, const int* __restrict__ bt, long bt_sr, const int* __restrict__ sl, int n_req,
    const int* __restrict__ rows, int n_rows, int max_fin, int page, int NB,
    const uint64_t* __restrict__ k_layers, long k_sb, long k_st, long k_sh, int n_kv,
    const uint16_t* __restrict__ tag, long layer_rows, uint8_t* __restrict__ mark,
    int* __restrict__ count)
{
    const long i = (long)blockIdx.x * RF_THREADS + threadIdx.x;
    if (i == 0 && blockIdx.y == 0) *count = 0;           // compact runs after this kernel
    // delta: one thread per (page, kv head), heads of one page adjacent
    const int kh = mode == LOCKS_REFRESH_DELTA ? (int)(i % n_kv) : 0;
    const long pi = mode == LOCKS_REFRESH_DELTA ? i / n_kv : i;
    int blk;
    if (mode == LOCKS_REFRESH_TAIL) {
        if (pi >= n_rows) return;
        const int r = rows ? rows[pi] : (int)pi;
        if (r < 0 || r >= n_req) return;
        const int fin1 = min(max(sl[r] / page - 1, 0), (int)bt_sr - 1);   // last finalized page
        blk = bt[(long)r * bt_sr + fin1];
    } else {
        if (pi >= (long)n_req * max_fin) return;
        const int r = (int)(pi / max_fin), p = (int)(pi % max_fin);
        if (p >= sl[r] / page) return;                    // not finalized
        blk = bt[(long)r * bt_sr + p];
    }
    if (blk < 0 || blk >= NB) return;
    if (mode == LOCKS_REFRESH_DELTA) {
        const int layer = blockIdx.y;
        const uint16_t* kp = reinterpret_cast<const uint16_t*>(k_layers[layer]) +
                             (long)blk * k_sb + (long)(page - 1) * k_st + (long)kh * k_sh;
        const uint16_t* tp = tag + ((long)layer * layer_rows + (long)blk * n_kv + kh) * 8;
        if (!tags_differ(*reinterpret_cast<const uint4*>(kp), *reinterpret_cast<const uint4*>(tp)))
            return;
    }
    mark[blk] = 1;
}

__global__ __launch_bounds__(RF_THREADS) void refresh_compact_kernel(
    uint8_t* __restrict__ mark, int NB, int* __restrict__ blocks, int* __restrict__ count)
{
    const int i = blockIdx.x * RF_THREADS + threadIdx.x;
    const int lane = threadIdx.x & 63;
    const bool m = i < NB && mark[i] != 0;
    if (m) mark[i] = 0;
    const uint64_t bal = __ballot(m);
    if (bal == 0) return;
    const int pre = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                              __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
    int base = 0;
    if (lane == 0) base = atomicAdd(count, __popcll(bal));
    base = __shfl(base, 0);
    if (m) blocks[base + pre] = i;
}

}  // namespace locks

using namespace locks;

// (head_dim, page) of the summary builder: {64, 128, 256} x {16, 32, 64}
// (the reference's rki4 geometry domain, rki4_state.py:295-324) plus the MLA
// latent (512, 16).
static bool bd_geometry(int head_dim, int page) {
    if (head_dim == 512) return page == 16;
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && (page == 16 || page == 32 || page == 64);
}
template <int D, int PG>
static int bd_launch(const uint16_t* kc, const uint64_t* k_layers, long k_sb, long k_st, long k_sh,
                     int NB, const int* blocks, const int* count, int n_blocks, int n_kv,
                     int n_layers, long layer_rows, const SlabRows& S, uint16_t* tag, hipStream_t st) {
    constexpr int nw = bd_waves<D, PG>();
    const long items = (long)n_blocks * n_kv * n_layers;
    const long grid = std::min((items + nw - 1) / nw, BD_MAX_GRID);
    hipLaunchKernelGGL((rki4_build_kernel<D, PG>), dim3((unsigned)grid), dim3(nw * kWave), 0, st,
                       kc, k_layers, k_sb, k_st, k_sh, NB, blocks, count, n_blocks, n_kv,
                       n_layers, layer_rows, S, tag);
    return check_launch("rki4_build_kernel");
}
#define BD_DISPATCH(HD, PGV, ...)                                              \
    ((HD) == 512 ? bd_launch<512, 16>(__VA_ARGS__)                               \
     : (PGV) == 16 ? ((HD) == 128 ? bd_launch<128, 16>(__VA_ARGS__)              \
                      : (HD) == 64 ? bd_launch<64, 16>(__VA_ARGS__)              \
                                   : bd_launch<256, 16>(__VA_ARGS__))            \
     : (PGV) == 32 ? ((HD) == 128 ? bd_launch<128, 32>(__VA_ARGS__)              \
                      : (HD) == 64 ? bd_launch<64, 32>(__VA_ARGS__)              \
                                   : bd_launch<256, 32>(__VA_ARGS__))            \
                   : ((HD) == 128 ? bd_launch<128, 64>(__VA_ARGS__)              \
                      : (HD) == 64 ? bd_launch<64, 64>(__VA_ARGS__)              \
                                   : bd_launch<256, 64>(__VA_ARGS__)))

extern "C" int32_t locks_build_rki4(
    const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok, int64_t k_stride_head,
    int32_t num_blocks, const int32_t* blocks, int32_t n_blocks, int32_t n_kv, int32_t head_dim,
    int32_t page, uint8_t* v4, uint16_t* vs, int8_t* c8, uint16_t* cs, int8_t* mu8,
    uint16_t* mus, const int64_t* slab_row_bytes, uint16_t* tag, void* stream)
{
    LOCKS_REQUIRE(bd_geometry(head_dim, page),
                  "locks_build_rki4: geometry d=%d page=%d unsupported (d 64/128/256 with page 16/32/64, "
                  "or d 512 with page 16)", head_dim, page);
    LOCKS_REQUIRE(n_kv >= 1 && num_blocks >= 1 && n_blocks >= 0, "locks_build_rki4: bad geometry");
    LOCKS_REQUIRE(k_stride_tok % 8 == 0 && k_stride_block % 8 == 0 && k_stride_head % 8 == 0,
                  "locks_build_rki4: K strides must be multiples of 8 elements");
    LOCKS_REQUIRE(k_cache && blocks && v4 && vs && c8 && cs && mu8 && mus && tag,
                  "locks_build_rki4: null pointer argument");
    const SlabRows S = slab_rows(v4, vs, c8, cs, mu8, mus, slab_row_bytes, head_dim, page);
    LOCKS_REQUIRE(slab_rows_ok(S, head_dim, page),
                  "locks_build_rki4: slab row strides below the field sizes or misaligned");
    if (n_blocks == 0) return 0;
    return BD_DISPATCH(head_dim, page, k_cache, nullptr, (long)k_stride_block, (long)k_stride_tok,
                       (long)k_stride_head, num_blocks, blocks, nullptr, n_blocks, n_kv, 1, 0L,
                       S, tag, (hipStream_t)stream);
}

extern "C" int32_t locks_pack_rki4(const float* mu, const float* dc, const float* S2,
                                   const float* U, const int32_t* rows, int32_t n,
                                   int32_t head_dim, int32_t page, uint8_t* v4, uint16_t* vs,
                                   int8_t* c8, uint16_t* cs, int8_t* mu8, uint16_t* mus,
                                   const int64_t* slab_row_bytes, void* stream)
{
    LOCKS_REQUIRE(head_dim == 128 && page == 16,
                  "locks_pack_rki4: geometry d=%d page=%d unsupported (this entry: 128/16)", head_dim, page);
    LOCKS_REQUIRE(n >= 0, "locks_pack_rki4: n=%d < 0", n);
    LOCKS_REQUIRE(mu && dc && S2 && U && rows && v4 && vs && c8 && cs && mu8 && mus,
                  "locks_pack_rki4: null pointer argument");
    const SlabRows S = slab_rows(v4, vs, c8, cs, mu8, mus, slab_row_bytes, head_dim, page);
    LOCKS_REQUIRE(slab_rows_ok(S, head_dim, page),
                  "locks_pack_rki4: slab row strides below the field sizes or misaligned");
    if (n == 0) return 0;
    hipLaunchKernelGGL(rki4_pack_kernel, dim3((n + 3) / 4), dim3(4 * kWave),
                       0, (hipStream_t)stream, mu, dc, S2, U, rows, n, S);
    return check_launch("rki4_pack_kernel");
}

extern "C" int32_t locks_refresh_blocks(
    int32_t mode, const int32_t* block_table, int64_t bt_stride, const int32_t* seq_lens,
    int32_t n_req, const int32_t* rows, int32_t n_rows, int32_t max_fin, int32_t page,
    int32_t num_blocks, const uint64_t* k_layers, int32_t n_layers, int64_t k_stride_block,
    int64_t k_stride_tok, int64_t k_stride_head, int32_t n_kv, const uint16_t* tag,
    int64_t tag_blocks, uint8_t* mark, int32_t* blocks, int32_t* count, void* stream)
{
    LOCKS_REQUIRE(mode == LOCKS_REFRESH_TAIL || mode == LOCKS_REFRESH_BULK ||
                      mode == LOCKS_REFRESH_DELTA,
                  "locks_refresh_blocks: unknown mode %d", mode);
    LOCKS_REQUIRE(block_table && seq_lens && mark && blocks && count,
                  "locks_refresh_blocks: null pointer argument");
    LOCKS_REQUIRE(n_req >= 0 && n_rows >= 0 && max_fin >= 0 && page >= 1 && num_blocks >= 1 &&
                      bt_stride >= 1,
                  "locks_refresh_blocks: bad geometry");
    if (mode == LOCKS_REFRESH_BULK || mode == LOCKS_REFRESH_DELTA)
        LOCKS_REQUIRE(max_fin <= bt_stride, "locks_refresh_blocks: max_fin %d > block-table width %lld",
                      max_fin, (long long)bt_stride);
    if (mode == LOCKS_REFRESH_DELTA) {
        LOCKS_REQUIRE(k_layers && tag && n_layers >= 1 && n_layers <= 65535 && n_kv >= 1 &&
                          tag_blocks >= num_blocks,
                      "locks_refresh_blocks: delta needs k_layers, tag, n_layers, n_kv");
        LOCKS_REQUIRE(k_stride_tok % 8 == 0 && k_stride_block % 8 == 0 && k_stride_head % 8 == 0,
                      "locks_refresh_blocks: K strides must be multiples of 8 elements");
    }
    const long items = mode == LOCKS_REFRESH_TAIL ? (long)n_rows
                       : (long)n_req * max_fin * (mode == LOCKS_REFRESH_DELTA ? n_kv : 1);
    const long gx = std::max<long>(1, (items + RF_THREADS - 1) / RF_THREADS);
    LOCKS_REQUIRE(gx < (1L << 31), "locks_refresh_blocks: too many pages in one call");
    const int gy = mode == LOCKS_REFRESH_DELTA ? n_layers : 1;
    hipLaunchKernelGGL(refresh_mark_kernel, dim3((unsigned)gx, gy), dim3(RF_THREADS), 0,
                       (hipStream_t)stream, mode, block_table, (long)bt_stride, seq_lens, n_req,
                       rows, n_rows, max_fin, page, num_blocks, k_layers, (long)k_stride_block,
                       (long)k_stride_tok, (long)k_stride_head, n_kv, tag,
                       (long)tag_blocks * n_kv, mark, count);
    int32_t rc = check_launch("refresh_mark_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(refresh_compact_kernel, dim3((num_blocks + RF_THREADS - 1) / RF_THREADS),
                       dim3(RF_THREADS), 0, (hipStream_t)stream, mark, num_blocks, blocks, count);
    return check_launch("refresh_compact_kernel");
}

extern "C" int32_t locks_build_rki4_layers(
    const uint64_t* k_layers, int32_t n_layers, int64_t k_stride_block, int64_t k_stride_tok,
    int64_t k_stride_head, int32_t num_blocks, const int32_t* blocks, const int32_t* count,
    int32_t n_blocks, int32_t n_kv, int32_t head_dim, int32_t page, int64_t slab_blocks,
    uint8_t* v4, uint16_t* vs, int8_t* c8, uint16_t* cs, int8_t* mu8, uint16_t* mus,
    const int64_t* slab_row_bytes, uint16_t* tag, void* stream)
{
    LOCKS_REQUIRE(bd_geometry(head_dim, page),
                  "locks_build_rki4_layers: geometry d=%d page=%d unsupported (d 64/128/256 with page "
                  "16/32/64, or d 512 with page 16)", head_dim, page);
    LOCKS_REQUIRE(n_kv >= 1 && num_blocks >= 1 && n_blocks >= 0 && n_layers >= 1 &&
                      n_layers <= 65535 && slab_blocks >= num_blocks,
                  "locks_build_rki4_layers: bad geometry");
    LOCKS_REQUIRE(k_stride_tok % 8 == 0 && k_stride_block % 8 == 0 && k_stride_head % 8 == 0,
                  "locks_build_rki4_layers: K strides must be multiples of 8 elements");
    LOCKS_REQUIRE(k_layers && blocks && v4 && vs && c8 && cs && mu8 && mus && tag,
                  "locks_build_rki4_layers: null pointer argument");
    const SlabRows S = slab_rows(v4, vs, c8, cs, mu8, mus, slab_row_bytes, head_dim, page);
    LOCKS_REQUIRE(slab_rows_ok(S, head_dim, page),
                  "locks_build_rki4_layers: slab row strides below the field sizes or misaligned");
    if (n_blocks == 0) return 0;
    const long layer_rows = (long)slab_blocks * n_kv;
    return BD_DISPATCH(head_dim, page, nullptr, k_layers, (long)k_stride_block, (long)k_stride_tok,
                       (long)k_stride_head, num_blocks, blocks, count, n_blocks, n_kv, n_layers,
                       layer_rows, S, tag, (hipStream_t)stream);
}
