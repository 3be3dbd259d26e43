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
#include "locks_common.h"
#include "locks_hip.h"

namespace locks {

constexpr int BD_PG = 16;
constexpr int BD_RNK = 8;
constexpr int BD_SWEEPS = 12;
// waves per workgroup: the per-wave LDS image of a d = 512 page is ~37 KB
template <int D> constexpr int bd_waves() { return D <= 128 ? 4 : 1; }

template <int D>
struct WaveLds {
    float dc[BD_PG][D + 1];      // centred page (padded rows)
    float mu[D];
    float A[BD_PG][BD_PG + 1];   // gram, rotated in place
    float U[BD_PG][BD_PG + 1];   // accumulated eigenvectors (columns)
    float cc[BD_PG], ss[BD_PG];
    int partner[BD_PG];
    float S8[BD_RNK];
    int col[BD_RNK];             // eigen column of basis r (ascending top-8)
    float red[BD_RNK][kWave / 8];
};

// quantize + pack one page from mu (LDS), dc (LDS), U8 = U[:, col[r]],
// S8 (LDS), writing the six slab rows.  Lane l owns the packed bytes
// j = l + 64 k (d = 2j, 2j + 1).
template <int D>
__device__ void pack_page(WaveLds<D>& L, long row, uint8_t* __restrict__ v4, uint16_t* __restrict__ vs,
                          int8_t* __restrict__ c8, uint16_t* __restrict__ cs,
                          int8_t* __restrict__ mu8, uint16_t* __restrict__ mus) {
    constexpr int NK = D / 128;
    const int lane = threadIdx.x & 63;
    // V[d][r]: sequential over t, separately rounded
    float V[NK][2][BD_RNK];
#pragma unroll
    for (int k = 0; k < NK; ++k)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int d = 2 * (lane + 64 * k) + e;
#pragma unroll
            for (int r = 0; r < BD_RNK; ++r) {
                float acc = 0.f;
                const int c = L.col[r];
                for (int t = 0; t < BD_PG; ++t) acc = __fadd_rn(acc, __fmul_rn(L.dc[t][d], L.U[t][c]));
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
    uint8_t* vrow = v4 + row * (BD_RNK * D / 2);
#pragma unroll
    for (int r = 0; r < BD_RNK; ++r)
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int lo = (int)fminf(fmaxf(rintf(__fdiv_rn(V[k][0][r], vsc[r])), -8.f), 7.f);
            const int hi = (int)fminf(fmaxf(rintf(__fdiv_rn(V[k][1][r], vsc[r])), -8.f), 7.f);
            vrow[r * (D / 2) + lane + 64 * k] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
        }
    if (lane < BD_RNK) vs[row * BD_RNK + lane] = f32_to_bf16(vsc[lane]);
    // coefficients: lane t < 16 owns token t
    if (lane < BD_PG) {
        const int t = lane;
        float C[BD_RNK];
        float am = 0.f;
#pragma unroll
        for (int r = 0; r < BD_RNK; ++r) {
            C[r] = __fmul_rn(L.U[t][L.col[r]], L.S8[r]);
            am = fmaxf(am, fabsf(C[r]));
        }
        const float csc = fmaxf(__fdiv_rn(am, 127.f), 1e-8f);
        int8_t* crow = c8 + (row * BD_PG + t) * BD_RNK;
#pragma unroll
        for (int r = 0; r < BD_RNK; ++r)
            crow[r] = (int8_t)fminf(fmaxf(rintf(__fdiv_rn(C[r], csc)), -127.f), 127.f);
        cs[row * BD_PG + t] = f32_to_bf16(csc);
    }
    // centroid
    float am = 0.f;
#pragma unroll
    for (int k = 0; k < NK; ++k)
        am = fmaxf(am, fmaxf(fabsf(L.mu[2 * (lane + 64 * k)]), fabsf(L.mu[2 * (lane + 64 * k) + 1])));
    am = wave_max(am);
    const float msc = fmaxf(__fdiv_rn(am, 127.f), 1e-8f);
#pragma unroll
    for (int k = 0; k < NK; ++k)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int d = 2 * (lane + 64 * k) + e;
            mu8[row * D + d] = (int8_t)fminf(fmaxf(rintf(__fdiv_rn(L.mu[d], msc)), -127.f), 127.f);
        }
    if (lane == 0) mus[row] = f32_to_bf16(msc);
}

// Parallel cyclic Jacobi on L.A (16x16 symmetric); eigenvectors -> L.U columns.
template <class W>
__device__ void jacobi16(W& L) {
    const int lane = threadIdx.x & 63;
    for (int i = lane; i < BD_PG * BD_PG; i += kWave) L.U[i / BD_PG][i % BD_PG] = (i / BD_PG == i % BD_PG) ? 1.f : 0.f;
    wave_lds_sync();
    for (int sweep = 0; sweep < BD_SWEEPS; ++sweep) {
        // convergence test: off-diagonal mass vs diagonal
        float off = 0.f, dia = 0.f;
        for (int i = lane; i < BD_PG * BD_PG; i += kWave) {
            const float a = L.A[i / BD_PG][i % BD_PG];
            if (i / BD_PG == i % BD_PG) dia += a * a; else off += a * a;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            off += __shfl_xor(off, o, kWave);
            dia += __shfl_xor(dia, o, kWave);
        }
        if (!(off > 1e-14f * dia) ) break;      // wave-uniform (also exits on 0/0)
        for (int step = 0; step < BD_PG - 1; ++step) {
            // round-robin pairing: index 0 fixed, 1..15 rotate
            if (lane < BD_PG / 2) {
                auto at = [&](int k) { return 1 + ((k + step) % (BD_PG - 1)); };
                const int p = lane == 0 ? 0 : at(lane);
                const int q = lane == 0 ? at(0) : at(BD_PG - 1 - lane);
                const float apq = L.A[p][q];
                float c = 1.f, s = 0.f;
                if (apq != 0.f) {
                    const float theta = (L.A[q][q] - L.A[p][p]) / (2.f * apq);
                    const float t = copysignf(1.f, theta) / (fabsf(theta) + sqrtf(theta * theta + 1.f));
                    c = 1.f / sqrtf(t * t + 1.f);
                    s = t * c;
                }
                L.cc[p] = c; L.ss[p] = -s; L.partner[p] = q;
                L.cc[q] = c; L.ss[q] = s;  L.partner[q] = p;
            }
            wave_lds_sync();
            // rows: A'[i][j] = cc[i] A[i][j] + ss[i] A[partner i][j]
            float nv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int idx = lane + e * kWave, i = idx / BD_PG, j = idx % BD_PG;
                nv[e] = L.cc[i] * L.A[i][j] + L.ss[i] * L.A[L.partner[i]][j];
            }
            wave_lds_sync();
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int idx = lane + e * kWave;
                L.A[idx / BD_PG][idx % BD_PG] = nv[e];
            }
            wave_lds_sync();
            // columns of A and of U
            float na[4], nu[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int idx = lane + e * kWave, i = idx / BD_PG, j = idx % BD_PG;
                na[e] = L.cc[j] * L.A[i][j] + L.ss[j] * L.A[i][L.partner[j]];
                nu[e] = L.cc[j] * L.U[i][j] + L.ss[j] * L.U[i][L.partner[j]];
            }
            wave_lds_sync();
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int idx = lane + e * kWave;
                L.A[idx / BD_PG][idx % BD_PG] = na[e];
                L.U[idx / BD_PG][idx % BD_PG] = nu[e];
            }
            wave_lds_sync();
        }
    }
}

// eigenvalues on the diagonal of L.A -> ascending ranks -> top-8 columns
template <class W>
__device__ void select_top8(W& L) {
    const int lane = threadIdx.x & 63;
    if (lane < BD_PG) {
        const float li = L.A[lane][lane];
        int rank = 0;
        for (int j = 0; j < BD_PG; ++j) {
            const float lj = L.A[j][j];
            rank += (lj < li) || (lj == li && j < lane);
        }
        if (rank >= BD_PG - BD_RNK) {
            const int r = rank - (BD_PG - BD_RNK);
            L.col[r] = lane;
            L.S8[r] = __fsqrt_rn(fmaxf(li, 1e-10f));
        }
    }
    wave_lds_sync();
}

template <int D>
__global__ __launch_bounds__(bd_waves<D>() * kWave) void rki4_build_kernel(
    const uint16_t* __restrict__ kc, long k_sb, long k_st, long k_sh, int NB,
    const int* __restrict__ blocks, int n_blocks, int n_kv,
    uint8_t* __restrict__ v4, uint16_t* __restrict__ vs, int8_t* __restrict__ c8,
    uint16_t* __restrict__ cs, int8_t* __restrict__ mu8, uint16_t* __restrict__ mus,
    uint16_t* __restrict__ tag)
{
    constexpr int NW = bd_waves<D>();
    __shared__ WaveLds<D> lds[NW];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    WaveLds<D>& L = lds[wave];
    const long item = (long)blockIdx.x * NW + wave;      // (block index, kv head)
    if (item >= (long)n_blocks * n_kv) return;
    const int bi = (int)(item / n_kv), kh = (int)(item % n_kv);
    const int blk = blocks[bi];
    if (blk < 0 || blk >= NB) return;                          // masked (profile pass)
    const long row = (long)blk * n_kv + kh;
    const uint16_t* kp = kc + (long)blk * k_sb + (long)kh * k_sh;

    // stage K (fp32) and the centroid (sequential sum over t, then / 16)
    for (int i = lane; i < BD_PG * D / 8; i += kWave) {
        const int t = i / (D / 8), d0 = (i % (D / 8)) * 8;
        const uint4 w = *reinterpret_cast<const uint4*>(kp + (long)t * k_st + d0);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            L.dc[t][d0 + 2 * e] = bf16lo(ws[e]);
            L.dc[t][d0 + 2 * e + 1] = bf16hi(ws[e]);
        }
    }
    if (lane < 8) tag[row * 8 + lane] = kp[(long)(BD_PG - 1) * k_st + lane];
    wave_lds_sync();
    for (int d = lane; d < D; d += kWave) {
        float acc = 0.f;
        for (int t = 0; t < BD_PG; ++t) acc = __fadd_rn(acc, L.dc[t][d]);
        const float m = __fdiv_rn(acc, (float)BD_PG);
        L.mu[d] = m;
        for (int t = 0; t < BD_PG; ++t) L.dc[t][d] = __fsub_rn(L.dc[t][d], m);
    }
    wave_lds_sync();

    // gram on the matrix core: Gm[i][j] = sum_d dc[i][d] dc[j][d]
    {
        const int i = lane & 15, kq = lane >> 4;
        v4f g = {0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < D / 4; ++s) {
            const float a = L.dc[i][4 * s + kq];
            g = __builtin_amdgcn_mfma_f32_16x16x4f32(a, a, g, 0, 0, 0);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) L.A[4 * kq + v][i] = g[v];
    }
    wave_lds_sync();
    jacobi16(L);
    select_top8(L);
    pack_page<D>(L, row, v4, vs, c8, cs, mu8, mus);
}

// locks_pack_rki4: quantize + pack given the caller's eigen decomposition.
__global__ __launch_bounds__(4 * kWave) void rki4_pack_kernel(
    const float* __restrict__ mu, const float* __restrict__ dc, const float* __restrict__ S2,
    const float* __restrict__ U, const int* __restrict__ rows, int n,
    uint8_t* __restrict__ v4, uint16_t* __restrict__ vs, int8_t* __restrict__ c8,
    uint16_t* __restrict__ cs, int8_t* __restrict__ mu8, uint16_t* __restrict__ mus)
{
    constexpr int BD_D = 128;
    __shared__ WaveLds<BD_D> lds[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    WaveLds<BD_D>& L = lds[wave];
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
    pack_page<BD_D>(L, rows[item], v4, vs, c8, cs, mu8, mus);
}

}  // namespace locks

using namespace locks;

extern "C" int32_t locks_build_rki4(
    const uint16_t* k_cache, int64_t k_stride_block, int64_t k_stride_tok, int64_t k_stride_head,
    int32_t num_blocks, const int32_t* blocks, int32_t n_blocks, int32_t n_kv, int32_t head_dim,
    int32_t page, uint8_t* v4, uint16_t* vs, int8_t* c8, uint16_t* cs, int8_t* mu8,
    uint16_t* mus, uint16_t* tag, void* stream)
{
    LOCKS_REQUIRE((head_dim == 128 || head_dim == 512) && page == BD_PG,
                  "locks_build_rki4: geometry d=%d page=%d unsupported (this build: d 128 or 512, page 16)",
                  head_dim, page);
    LOCKS_REQUIRE(n_kv >= 1 && num_blocks >= 1 && n_blocks >= 0, "locks_build_rki4: bad geometry");
    LOCKS_REQUIRE(k_stride_tok % 8 == 0 && k_stride_block % 8 == 0 && k_stride_head % 8 == 0,
                  "locks_build_rki4: K strides must be multiples of 8 elements");
    LOCKS_REQUIRE(k_cache && blocks && v4 && vs && c8 && cs && mu8 && mus && tag,
                  "locks_build_rki4: null pointer argument");
    if (n_blocks == 0) return 0;
    const long items = (long)n_blocks * n_kv;
    const int nw = head_dim == 128 ? bd_waves<128>() : bd_waves<512>();
    const long grid = (items + nw - 1) / nw;
    LOCKS_REQUIRE(grid < (1L << 31), "locks_build_rki4: too many pages in one call");
#define BUILD_LAUNCH(DV)                                                                     \
    hipLaunchKernelGGL((rki4_build_kernel<DV>), dim3((unsigned)grid), dim3(nw * kWave), 0,  \
                       (hipStream_t)stream, k_cache, (long)k_stride_block, (long)k_stride_tok, \
                       (long)k_stride_head, num_blocks, blocks, n_blocks, n_kv, v4, vs, c8, cs, \
                       mu8, mus, tag)
    if (head_dim == 128) BUILD_LAUNCH(128);
    else BUILD_LAUNCH(512);
#undef BUILD_LAUNCH
    return check_launch("rki4_build_kernel");
}

extern "C" int32_t locks_pack_rki4(const float* mu, const float* dc, const float* S2,
                                   const float* U, const int32_t* rows, int32_t n,
                                   int32_t head_dim, int32_t page, uint8_t* v4, uint16_t* vs,
                                   int8_t* c8, uint16_t* cs, int8_t* mu8, uint16_t* mus,
                                   void* stream)
{
    LOCKS_REQUIRE(head_dim == 128 && page == BD_PG,
                  "locks_pack_rki4: geometry d=%d page=%d unsupported (this build: 128/16)", head_dim, page);
    LOCKS_REQUIRE(n >= 0, "locks_pack_rki4: n=%d < 0", n);
    LOCKS_REQUIRE(mu && dc && S2 && U && rows && v4 && vs && c8 && cs && mu8 && mus,
                  "locks_pack_rki4: null pointer argument");
    if (n == 0) return 0;
    hipLaunchKernelGGL(rki4_pack_kernel, dim3((n + 3) / 4), dim3(4 * kWave),
                       0, (hipStream_t)stream, mu, dc, S2, U, rows, n, v4, vs, c8, cs, mu8, mus);
    return check_launch("rki4_pack_kernel");
}
