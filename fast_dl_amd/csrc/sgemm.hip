// fp32 GEMM kernels for gfx950 (CDNA4) built on the fp32 matrix-core
// instruction v_mfma_f32_32x32x2_f32, plus a VALU strip kernel for skinny
// shapes.  The reference ran this product through cublasSgemm in pedantic
// fp32 (src/kernels/cuda/gemm.cu:166-177); the arithmetic here is also plain
// fp32 multiply-add with fp32 accumulation, only the summation order differs.
//
// MFMA 32x32x2 lane layout (wave64), used by every kernel below:
//   operand a: lane l supplies A[i = l % 32][kk = l / 32]
//   operand b: lane l supplies B[kk = l / 32][j = l % 32]
//   result   : lane l, register r holds D[i][j] with j = l % 32 and
//              i = 8 * (r / 4) + 4 * (l / 32) + (r % 4)
#include "fdl_internal.hpp"

#include <algorithm>

namespace fdl {

namespace {

constexpr int kWave = 64;

// The GPU hands workgroups to its 8 XCDs round-robin (workgroup b runs on
// XCD b % 8) and each XCD has its own L2.  Renumber so each XCD owns one
// contiguous range of logical tiles, then walk that range in groups of G tile
// rows so the tiles resident on one XCD share A row-panels and B col-panels.
__device__ __forceinline__ void tile_coords(int bid, int nblocks, int tiles_m,
                                            int tiles_n, int& tm, int& tn) {
    if ((nblocks & 7) == 0) {
        bid = (bid & 7) * (nblocks >> 3) + (bid >> 3);
    }
    constexpr int G = 8;
    const int width = G * tiles_n;
    const int group = bid / width;
    const int first_m = group * G;
    const int gsize = min(tiles_m - first_m, G);
    const int in_group = bid - group * width;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

__device__ __forceinline__ float apply_epilogue(float v, int epi,
                                                const float* __restrict__ bias,
                                                const float* __restrict__ aux,
                                                int64_t c_off, int j) {
    switch (epi) {
        case EPI_BIAS:
            return v + bias[j];
        case EPI_BIAS_RELU:
            return fmaxf(0.0f, v + bias[j]);
        case EPI_RELU:
            return fmaxf(0.0f, v);
        case EPI_RELU_GRAD:
            return aux[c_off] > 0.0f ? v : 0.0f;
        default:
            return v;
    }
}

// ---------------------------------------------------------------------------
// Global -> register -> LDS tile staging.
//
// A tile covers MN rows (m or n) by BK reduction steps.  In LDS it is always
// stored k-major, [BK][MN + PAD], so that the MFMA operand read (32 lanes on
// 32 consecutive m/n at one k) is one conflict-free ds_read_b32 per half-wave.
// KCONTIG says how the operand sits in global memory: element (mn, k) is at
// p[mn * ld + k] when KCONTIG (A not transposed, B transposed), else at
// p[k * ld + mn].  VEC uses 16-byte loads along the contiguous dimension; the
// host only selects it when that dimension and ld are multiples of 4 and the
// base is 16-byte aligned, so a float4 is either wholly inside or wholly
// outside the matrix.
// ---------------------------------------------------------------------------
template <int MN, int BK, int NT, int PAD, bool KCONTIG, bool VEC>
struct TileLoader {
    static constexpr int LD = MN + PAD;
    static constexpr int VW = VEC ? 4 : 1;
    static constexpr int SLOTS = MN * BK / (VW * NT);
    static_assert(SLOTS * VW * NT == MN * BK, "tile must divide evenly");
    static constexpr int PER = KCONTIG ? BK / VW : MN / VW;  // slots per row
    float r[SLOTS * VW];

    __device__ __forceinline__ void coords(int idx, int& mn, int& k) const {
        if (KCONTIG) {
            mn = idx / PER;
            k = (idx % PER) * VW;
        } else {
            k = idx / PER;
            mn = (idx % PER) * VW;
        }
    }

    __device__ __forceinline__ void load(const float* __restrict__ p, int64_t ld,
                                         int mn_lim, int k_lim, int mn0, int k0,
                                         int tid, bool check) {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            int mn, k;
            coords(tid + s * NT, mn, k);
            const int gmn = mn0 + mn;
            const int gk = k0 + k;
            const bool ok = !check || (gmn < mn_lim && gk < k_lim);
            const int64_t off = KCONTIG ? (int64_t)gmn * ld + gk
                                        : (int64_t)gk * ld + gmn;
            if (VEC) {
                floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (ok) {
                    v = *reinterpret_cast<const floatx4*>(p + off);
                }
                r[4 * s + 0] = v[0];
                r[4 * s + 1] = v[1];
                r[4 * s + 2] = v[2];
                r[4 * s + 3] = v[3];
            } else {
                r[s] = ok ? p[off] : 0.0f;
            }
        }
    }

    __device__ __forceinline__ void store(float* __restrict__ lds, int tid) const {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            int mn, k;
            coords(tid + s * NT, mn, k);
            if (VEC && !KCONTIG) {
                floatx4 v = {r[4 * s + 0], r[4 * s + 1], r[4 * s + 2], r[4 * s + 3]};
                *reinterpret_cast<floatx4*>(lds + k * LD + mn) = v;
            } else if (VEC) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    lds[(k + j) * LD + mn] = r[4 * s + j];
                }
            } else {
                lds[k * LD + mn] = r[s];
            }
        }
    }
};

// ---------------------------------------------------------------------------
// LDS double-buffered MFMA tile kernel.  NT = 64 * (BM/WM) * (BN/WN) threads;
// each wave owns a WM x WN block of C made of (WM/32) x (WN/32) MFMA 32x32
// accumulators.  Per K-tile: the next tile's global loads are issued first,
// the current LDS buffer feeds the MFMAs, then the prefetched registers go to
// the other LDS buffer and one barrier closes the step.  PAD floats of padding
// per LDS row; WPE is the minimum number of waves per SIMD the register
// allocation must allow (occupancy target).
// ---------------------------------------------------------------------------
template <int BM_, int BN_, int BK_, int WM_, int WN_, int PAD_, int WPE_, int PRIO_ = 0>
struct TileCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int PAD = PAD_, WPE = WPE_, PRIO = PRIO_;
    static constexpr int NT = kWave * (BM / WM) * (BN / WN);
};

template <class Cfg, bool TA, bool TB, bool VA, bool VB>
__global__ void __launch_bounds__(Cfg::NT, Cfg::WPE)
sgemm_tiled_kernel(GemmParams p, int tiles_m, int tiles_n) {
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, WM = Cfg::WM, WN = Cfg::WN;
    constexpr int NT = Cfg::NT;
    constexpr int FM = WM / 32;
    constexpr int FN = WN / 32;
    constexpr int WGM = BM / WM;
    static_assert(BK % 2 == 0, "MFMA consumes k in pairs");

    using LoaderA = TileLoader<BM, BK, NT, Cfg::PAD, !TA, VA>;
    using LoaderB = TileLoader<BN, BK, NT, Cfg::PAD, TB, VB>;
    __shared__ __attribute__((aligned(16))) float As[2][BK * LoaderA::LD];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * LoaderB::LD];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int l32 = lane & 31;
    const int half = lane >> 5;
    const int wm0 = (wave % WGM) * WM;
    const int wn0 = (wave / WGM) * WN;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const int64_t bz = blockIdx.y;
    const float* __restrict__ A = p.A + bz * p.strideA;
    const float* __restrict__ B = p.B + bz * p.strideB;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int ni = 0; ni < FN; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;

    const bool edge_mn = (m0 + BM > p.M) || (n0 + BN > p.N);
    const int ktiles = (p.K + BK - 1) / BK;

    if (ktiles > 0) {
        LoaderA la;
        LoaderB lb;
        {
            const bool chk = edge_mn || (BK > p.K);
            la.load(A, p.lda, p.M, p.K, m0, 0, tid, chk);
            lb.load(B, p.ldb, p.N, p.K, n0, 0, tid, chk);
            la.store(As[0], tid);
            lb.store(Bs[0], tid);
        }
        __syncthreads();

        for (int t = 0; t < ktiles; ++t) {
            const int cur = t & 1;
            const bool has_next = (t + 1) < ktiles;
            if (has_next) {
                const int k0 = (t + 1) * BK;
                const bool chk = edge_mn || (k0 + BK > p.K);
                la.load(A, p.lda, p.M, p.K, m0, k0, tid, chk);
                lb.load(B, p.ldb, p.N, p.K, n0, k0, tid, chk);
            }
            const float* __restrict__ as = As[cur];
            const float* __restrict__ bs = Bs[cur];
            // Read every operand fragment of this K-tile before the first MFMA,
            // so the LDS latency is paid once per tile rather than per k pair.
            float a[BK / 2][FM];
            float b[BK / 2][FN];
#pragma unroll
            for (int kp = 0; kp < BK / 2; ++kp) {
#pragma unroll
                for (int mi = 0; mi < FM; ++mi)
                    a[kp][mi] = as[(2 * kp + half) * LoaderA::LD + wm0 + mi * 32 + l32];
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
                    b[kp][ni] = bs[(2 * kp + half) * LoaderB::LD + wn0 + ni * 32 + l32];
            }
            // Keep the scheduler from sinking the reads back next to their MFMAs.
            __builtin_amdgcn_sched_barrier(0);
            if (Cfg::PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int kp = 0; kp < BK / 2; ++kp)
#pragma unroll
                for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                    for (int ni = 0; ni < FN; ++ni)
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            a[kp][mi], b[kp][ni], acc[mi][ni], 0, 0, 0);
            if (Cfg::PRIO) __builtin_amdgcn_s_setprio(0);
            if (has_next) {
                la.store(As[cur ^ 1], tid);
                lb.store(Bs[cur ^ 1], tid);
            }
            __syncthreads();
        }
    }

    float* __restrict__ C = p.C + bz * p.strideC;
    const float* __restrict__ aux = p.aux ? p.aux + bz * p.strideC : nullptr;
    const int epi = p.epilogue;
    const bool has_bias = epi == EPI_BIAS || epi == EPI_BIAS_RELU;
    const bool relu = epi == EPI_BIAS_RELU || epi == EPI_RELU;
#pragma unroll
    for (int ni = 0; ni < FN; ++ni) {
        const int j = n0 + wn0 + ni * 32 + l32;
        const bool j_ok = j < p.N;
        // One bias value per lane and column block, loaded once.
        const float bj = (has_bias && j_ok) ? p.bias[j] : 0.0f;
#pragma unroll
        for (int mi = 0; mi < FM; ++mi) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = m0 + wm0 + mi * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (j_ok && i < p.M) {
                    const int64_t off = (int64_t)i * p.ldc + j;
                    float v = acc[mi][ni][r];
                    if (has_bias) v += bj;
                    if (relu) v = fmaxf(0.0f, v);
                    if (epi == EPI_RELU_GRAD) v = aux[off] > 0.0f ? v : 0.0f;
                    C[off] = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Small-problem kernel: one 32x32 tile of C per block, the K range split over
// KW waves.  Operands go straight from global (L2) into MFMA registers with
// the k index permuted inside each group of 8: at step s (0..3) the lane in
// half h supplies k = k0 + 4h + s, so one lane's four A values are contiguous
// (a 16-byte load when A is k-contiguous).  The permutation is applied to A
// and B alike, so the four MFMAs still cover k0..k0+7 exactly once.  Partial
// 32x32 sums meet in LDS and are added in wave order, then the epilogue runs.
// ---------------------------------------------------------------------------
template <int KW, bool TA, bool TB, bool VA, bool VB>
__global__ void __launch_bounds__(KW * 64)
sgemm_splitk32_kernel(GemmParams p, int tiles_m, int tiles_n, int kchunk) {
    __shared__ float red[KW][16][kWave];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int i = lane & 31;
    const int h = lane >> 5;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * 32;
    const int n0 = tn * 32;
    const int64_t bz = blockIdx.y;
    const float* __restrict__ A = p.A + bz * p.strideA;
    const float* __restrict__ B = p.B + bz * p.strideB;

    const int row = m0 + i;  // row of op(A) this lane feeds
    const int col = n0 + i;  // column of op(B) this lane feeds
    const bool row_ok = row < p.M;
    const bool col_ok = col < p.N;
    const int kbeg = wave * kchunk;
    const int kend = min(p.K, kbeg + kchunk);

    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

    for (int k = kbeg; k < kend; k += 8) {
        const int kb = k + 4 * h;
        float a[4];
        float b[4];
        if (k + 8 <= kend) {
            if (!TA) {
                const float* ar = A + (int64_t)row * p.lda + kb;
                if (VA) {
                    floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
                    if (row_ok) v = *reinterpret_cast<const floatx4*>(ar);
                    a[0] = v[0]; a[1] = v[1]; a[2] = v[2]; a[3] = v[3];
                } else {
#pragma unroll
                    for (int s = 0; s < 4; ++s) a[s] = row_ok ? ar[s] : 0.0f;
                }
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    a[s] = row_ok ? A[(int64_t)(kb + s) * p.lda + row] : 0.0f;
            }
            if (TB) {
                const float* br = B + (int64_t)col * p.ldb + kb;
                if (VB) {
                    floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
                    if (col_ok) v = *reinterpret_cast<const floatx4*>(br);
                    b[0] = v[0]; b[1] = v[1]; b[2] = v[2]; b[3] = v[3];
                } else {
#pragma unroll
                    for (int s = 0; s < 4; ++s) b[s] = col_ok ? br[s] : 0.0f;
                }
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    b[s] = col_ok ? B[(int64_t)(kb + s) * p.ldb + col] : 0.0f;
            }
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int kk = kb + s;
                const bool kin = kk < kend;
                a[s] = (row_ok && kin)
                           ? (TA ? A[(int64_t)kk * p.lda + row] : A[(int64_t)row * p.lda + kk])
                           : 0.0f;
                b[s] = (col_ok && kin)
                           ? (TB ? B[(int64_t)col * p.ldb + kk] : B[(int64_t)kk * p.ldb + col])
                           : 0.0f;
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], acc, 0, 0, 0);
    }

#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();

    float* __restrict__ C = p.C + bz * p.strideC;
    const float* __restrict__ aux = p.aux ? p.aux + bz * p.strideC : nullptr;
    for (int e = tid; e < 16 * kWave; e += KW * kWave) {
        const int r = e / kWave;
        const int ln = e % kWave;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < KW; ++w) v += red[w][r][ln];
        const int gi = m0 + 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3);
        const int gj = n0 + (ln & 31);
        if (gi < p.M && gj < p.N) {
            const int64_t off = (int64_t)gi * p.ldc + gj;
            C[off] = apply_epilogue(v, p.epilogue, p.bias, aux, off, gj);
        }
    }
}

// ---------------------------------------------------------------------------
// Skinny kernel for M <= MR (MR <= 8) with B not transposed: a bandwidth
// kernel whose cost is one pass over B.  A block owns a strip of 16 columns
// and the whole K range: CL lanes across the strip (4 lanes x float4 when VB,
// else 16 lanes x 1) and KL = 256 / CL lanes along K.  Each lane keeps MR x CW
// partial sums in registers; the KL partials meet in LDS and are added in
// lane order.  Strips are renumbered so the 8 XCDs each stream one
// contiguous band of B's columns (neighbouring strips share 128-byte lines).
// ---------------------------------------------------------------------------
template <int MR, bool TA, bool VB>
__global__ void __launch_bounds__(256)
sgemm_skinny_kernel(GemmParams p, int strips) {
    constexpr int NT = 256;
    constexpr int STRIP = 16;
    constexpr int CW = VB ? 4 : 1;
    constexpr int CL = STRIP / CW;
    constexpr int KL = NT / CL;
    __shared__ float red[KL][MR][STRIP];

    const int tid = threadIdx.x;
    const int cl = tid % CL;
    const int kl = tid / CL;

    int sid = blockIdx.x;
    if ((strips & 7) == 0) sid = (sid & 7) * (strips >> 3) + (sid >> 3);
    const int n0 = sid * STRIP + cl * CW;
    const int64_t bz = blockIdx.y;
    const float* __restrict__ A = p.A + bz * p.strideA;
    const float* __restrict__ B = p.B + bz * p.strideB;
    const bool col_ok = n0 < p.N;  // VB: N % 4 == 0, so the float4 is whole

    float acc[MR][CW];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < CW; ++c) acc[m][c] = 0.0f;

    const int M = p.M;
#pragma unroll 4
    for (int k = kl; k < p.K; k += KL) {
        float b[CW];
        if (VB) {
            floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (col_ok) v = *reinterpret_cast<const floatx4*>(B + (int64_t)k * p.ldb + n0);
#pragma unroll
            for (int c = 0; c < CW; ++c) b[c] = v[c];
        } else {
            b[0] = col_ok ? B[(int64_t)k * p.ldb + n0] : 0.0f;
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float a = 0.0f;
            if (m < M) a = TA ? A[(int64_t)k * p.lda + m] : A[(int64_t)m * p.lda + k];
#pragma unroll
            for (int c = 0; c < CW; ++c) acc[m][c] = fmaf(a, b[c], acc[m][c]);
        }
    }

#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < CW; ++c) red[kl][m][cl * CW + c] = acc[m][c];
    __syncthreads();

    float* __restrict__ C = p.C + bz * p.strideC;
    const float* __restrict__ aux = p.aux ? p.aux + bz * p.strideC : nullptr;
    for (int e = tid; e < MR * STRIP; e += NT) {
        const int m = e / STRIP;
        const int c = e % STRIP;
        const int j = sid * STRIP + c;
        if (m < M && j < p.N) {
            float v = 0.0f;
            for (int q = 0; q < KL; ++q) v += red[q][m][c];
            const int64_t off = (int64_t)m * p.ldc + j;
            C[off] = apply_epilogue(v, p.epilogue, p.bias, aux, off, j);
        }
    }
}

// ---------------------------------------------------------------------------
// Host-side launchers.
// ---------------------------------------------------------------------------

inline bool aligned16(const void* ptr) {
    return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0;
}

// 16-byte loads along an operand's contiguous dimension are safe when that
// dimension, the leading dimension and the batch stride are multiples of 4
// and the base pointer is 16-byte aligned.
inline bool vec_ok(const float* ptr, int64_t contig_extent, int64_t ld,
                   int64_t stride, int64_t batch) {
    return aligned16(ptr) && (contig_extent % 4 == 0) && (ld % 4 == 0) &&
           (batch <= 1 || stride % 4 == 0);
}

template <class Cfg>
hipError_t launch_tiled(const GemmParams& p, bool ta, bool tb, bool va, bool vb,
                        int nbatch, hipStream_t stream) {
    const int tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;
    const int tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    const dim3 grid(tiles_m * tiles_n, nbatch);
    const dim3 block(Cfg::NT);
    const int code = (ta ? 8 : 0) | (tb ? 4 : 0) | (va ? 2 : 0) | (vb ? 1 : 0);
#define FDL_TILED_CASE(C, TA_, TB_, VA_, VB_)                                         \
    case C:                                                                           \
        hipLaunchKernelGGL((sgemm_tiled_kernel<Cfg, TA_, TB_, VA_, VB_>), grid, block, 0, \
                           stream, p, tiles_m, tiles_n);                            \
        break;
    switch (code) {
        FDL_TILED_CASE(0, false, false, false, false)
        FDL_TILED_CASE(1, false, false, false, true)
        FDL_TILED_CASE(2, false, false, true, false)
        FDL_TILED_CASE(3, false, false, true, true)
        FDL_TILED_CASE(4, false, true, false, false)
        FDL_TILED_CASE(5, false, true, false, true)
        FDL_TILED_CASE(6, false, true, true, false)
        FDL_TILED_CASE(7, false, true, true, true)
        FDL_TILED_CASE(8, true, false, false, false)
        FDL_TILED_CASE(9, true, false, false, true)
        FDL_TILED_CASE(10, true, false, true, false)
        FDL_TILED_CASE(11, true, false, true, true)
        FDL_TILED_CASE(12, true, true, false, false)
        FDL_TILED_CASE(13, true, true, false, true)
        FDL_TILED_CASE(14, true, true, true, false)
        FDL_TILED_CASE(15, true, true, true, true)
    }
#undef FDL_TILED_CASE
    return hipGetLastError();
}

hipError_t launch_splitk32(const GemmParams& p, bool ta, bool tb, bool va, bool vb,
                           int nbatch, hipStream_t stream) {
    constexpr int KW = 8;
    const int tiles_m = (p.M + 31) / 32;
    const int tiles_n = (p.N + 31) / 32;
    // K range per wave, a multiple of 8 (one MFMA group).
    int kchunk = (p.K + KW - 1) / KW;
    kchunk = std::max(8, (kchunk + 7) / 8 * 8);
    const dim3 grid(tiles_m * tiles_n, nbatch);
    const dim3 block(KW * kWave);
    // VA is only used for k-contiguous A (not transposed), VB only for
    // k-contiguous B (transposed); normalise to avoid dead instantiations.
    va = va && !ta;
    vb = vb && tb;
    const int code = (ta ? 8 : 0) | (tb ? 4 : 0) | (va ? 2 : 0) | (vb ? 1 : 0);
#define FDL_SPLITK_CASE(C, TA_, TB_, VA_, VB_)                                   \
    case C:                                                                      \
        hipLaunchKernelGGL((sgemm_splitk32_kernel<KW, TA_, TB_, VA_, VB_>), grid, \
                           block, 0, stream, p, tiles_m, tiles_n, kchunk);       \
        break;
    switch (code) {
        FDL_SPLITK_CASE(0, false, false, false, false)
        FDL_SPLITK_CASE(2, false, false, true, false)
        FDL_SPLITK_CASE(4, false, true, false, false)
        FDL_SPLITK_CASE(5, false, true, false, true)
        FDL_SPLITK_CASE(6, false, true, true, false)
        FDL_SPLITK_CASE(7, false, true, true, true)
        FDL_SPLITK_CASE(8, true, false, false, false)
        FDL_SPLITK_CASE(12, true, true, false, false)
        FDL_SPLITK_CASE(13, true, true, false, true)
        default:
            return hipErrorInvalidValue;
    }
#undef FDL_SPLITK_CASE
    return hipGetLastError();
}

template <int MR>
hipError_t launch_skinny_mr(const GemmParams& p, bool ta, bool vb, int nbatch,
                            hipStream_t stream) {
    const int strips = (p.N + 15) / 16;
    const dim3 grid(strips, nbatch);
    const dim3 block(256);
    if (ta) {
        if (vb) hipLaunchKernelGGL((sgemm_skinny_kernel<MR, true, true>), grid, block, 0, stream, p, strips);
        else hipLaunchKernelGGL((sgemm_skinny_kernel<MR, true, false>), grid, block, 0, stream, p, strips);
    } else {
        if (vb) hipLaunchKernelGGL((sgemm_skinny_kernel<MR, false, true>), grid, block, 0, stream, p, strips);
        else hipLaunchKernelGGL((sgemm_skinny_kernel<MR, false, false>), grid, block, 0, stream, p, strips);
    }
    return hipGetLastError();
}

hipError_t launch_skinny(const GemmParams& p, bool ta, bool vb, int nbatch,
                         hipStream_t stream) {
    if (p.M <= 1) return launch_skinny_mr<1>(p, ta, vb, nbatch, stream);
    if (p.M <= 2) return launch_skinny_mr<2>(p, ta, vb, nbatch, stream);
    if (p.M <= 4) return launch_skinny_mr<4>(p, ta, vb, nbatch, stream);
    return launch_skinny_mr<8>(p, ta, vb, nbatch, stream);
}

constexpr int kMaxGridY = 65535;

// Production tile configurations (BM, BN, BK, WM, WN, PAD, waves per SIMD).
using CfgTiled128 = TileCfg<128, 128, 16, 64, 64, 4, 1>;
using CfgTiled64 = TileCfg<64, 64, 16, 32, 32, 4, 1>;
using CfgTiled256 = TileCfg<256, 256, 16, 128, 64, 4, 1>;
using CfgTiled256x128 = TileCfg<256, 128, 16, 64, 64, 4, 1>;
using CfgTiled128W8 = TileCfg<128, 128, 16, 32, 64, 4, 1>;

// Dispatch cost model.  A config runs `slots` blocks per CU at full
// occupancy (LDS and register bound), each block holding `waves` waves; eff[w]
// is the measured fraction of fp32-MFMA peak a CU reaches with w resident
// waves per SIMD (w = 1..8).  The predicted time of a problem is the time of
// the most loaded CU: its tiles run in rounds of up to `slots` co-resident
// blocks, each round costing (tiles in round) * BM * BN / eff[w].
struct TileModel {
    GemmKernel kernel;
    int bm, bn, slots, waves;
    float eff[9];
};

constexpr TileModel kTileModels[] = {
    {GemmKernel::Tiled256, 256, 256, 1, 8, {0, 0.50f, 0.79f, 0.79f, 0.79f, 0.79f, 0.79f, 0.79f, 0.79f}},
    {GemmKernel::Tiled256x128, 256, 128, 2, 8, {0, 0.45f, 0.70f, 0.74f, 0.79f, 0.79f, 0.79f, 0.79f, 0.79f}},
    {GemmKernel::Tiled128, 128, 128, 3, 4, {0, 0.565f, 0.72f, 0.80f, 0.80f, 0.80f, 0.80f, 0.80f, 0.80f}},
    {GemmKernel::Tiled128W8, 128, 128, 3, 8, {0, 0.45f, 0.63f, 0.68f, 0.72f, 0.74f, 0.75f, 0.75f, 0.75f}},
    {GemmKernel::Tiled64, 64, 64, 8, 4, {0, 0.30f, 0.45f, 0.52f, 0.60f, 0.63f, 0.65f, 0.67f, 0.68f}},
};

double predicted_time(const TileModel& t, int M, int N, int64_t batch) {
    constexpr int64_t kCUs = 256;
    const int64_t tiles = (int64_t)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * batch;
    const int64_t per_cu = (tiles + kCUs - 1) / kCUs;
    const double work = (double)t.bm * t.bn;
    const int64_t full = per_cu / t.slots;
    const int64_t rest = per_cu % t.slots;
    auto round_cost = [&](int64_t blocks) {
        const int w = (int)std::min<int64_t>(8, std::max<int64_t>(1, blocks * t.waves / 4));
        return (double)blocks * work / t.eff[w];
    };
    double time = (double)full * round_cost(t.slots);
    if (rest) time += round_cost(rest);
    return time;
}

}  // namespace

const char* kernel_name(GemmKernel k) {
    switch (k) {
        case GemmKernel::Tiled128: return "tiled128";
        case GemmKernel::Tiled64: return "tiled64";
        case GemmKernel::SplitK32: return "splitk32";
        case GemmKernel::Skinny: return "skinny";
        case GemmKernel::Tiled256: return "tiled256";
        case GemmKernel::Tiled256x128: return "tiled256x128";
        case GemmKernel::Tiled128W8: return "tiled128w8";
        case GemmKernel::Auto: return "auto";
    }
    return "unknown";
}

GemmKernel choose_kernel(const GemmParams& p, bool transA, bool transB,
                         int64_t batch) {
    (void)transA;
    // Skinny M: one streaming pass over B on the VALU beats an MFMA tile
    // that would be at most 8/32 occupied.
    if (p.M <= 8 && !transB && p.N >= 64) return GemmKernel::Skinny;
    const int64_t t64 = (int64_t)((p.M + 63) / 64) * ((p.N + 63) / 64) * batch;
    constexpr int64_t kCUs = 256;
    // Too few 64x64 tiles to occupy the GPU, or too short a K loop to
    // amortise LDS staging: split K over the waves of a block instead.
    if (t64 < kCUs || p.K < 64) return GemmKernel::SplitK32;
    GemmKernel best = GemmKernel::Tiled64;
    double best_time = 0.0;
    bool first = true;
    for (const TileModel& t : kTileModels) {
        const double tm = predicted_time(t, p.M, p.N, batch);
        if (first || tm < best_time * 0.99) {  // ties keep the earlier (larger) tile
            best = t.kernel;
            best_time = tm;
            first = false;
        }
    }
    return best;
}

hipError_t launch_sgemm(const GemmParams& p0, bool transA, bool transB,
                        int64_t batch, GemmKernel kernel, hipStream_t stream) {
    if (batch <= 0 || p0.M <= 0 || p0.N <= 0) return hipSuccess;
    if (kernel == GemmKernel::Auto) kernel = choose_kernel(p0, transA, transB, batch);
    if (kernel == GemmKernel::Skinny && (transB || p0.M > 8)) return hipErrorInvalidValue;

    const bool va = vec_ok(p0.A, transA ? p0.M : p0.K, p0.lda, p0.strideA, batch);
    const bool vb = vec_ok(p0.B, transB ? p0.K : p0.N, p0.ldb, p0.strideB, batch);

    for (int64_t b0 = 0; b0 < batch; b0 += kMaxGridY) {
        const int nb = (int)std::min<int64_t>(kMaxGridY, batch - b0);
        GemmParams p = p0;
        p.A += b0 * p0.strideA;
        p.B += b0 * p0.strideB;
        p.C += b0 * p0.strideC;
        if (p.aux) p.aux += b0 * p0.strideC;
        hipError_t err = hipSuccess;
        switch (kernel) {
            case GemmKernel::Tiled128:
                err = launch_tiled<CfgTiled128>(p, transA, transB, va, vb, nb, stream);
                break;
            case GemmKernel::Tiled64:
                err = launch_tiled<CfgTiled64>(p, transA, transB, va, vb, nb, stream);
                break;
            case GemmKernel::Tiled256:
                err = launch_tiled<CfgTiled256>(p, transA, transB, va, vb, nb, stream);
                break;
            case GemmKernel::Tiled256x128:
                err = launch_tiled<CfgTiled256x128>(p, transA, transB, va, vb, nb, stream);
                break;
            case GemmKernel::Tiled128W8:
                err = launch_tiled<CfgTiled128W8>(p, transA, transB, va, vb, nb, stream);
                break;
            case GemmKernel::SplitK32:
                err = launch_splitk32(p, transA, transB, va, vb, nb, stream);
                break;
            case GemmKernel::Skinny:
                err = launch_skinny(p, transA, vb, nb, stream);
                break;
            default:
                return hipErrorInvalidValue;
        }
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

}  // namespace fdl
