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
#include "fdl_device.hpp"
#include "dma_loops.inc"
#include "fdl_internal.hpp"

#include <algorithm>
#include <type_traits>
#include <utility>

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

// Applies the epilogue to accumulator v of element (., j) at offset off and
// stores it.  EPI_SGD also updates the parameter: upd -= lr * v, with the
// product rounded before the subtraction as in the reference's host update.
__device__ __forceinline__ void store_epilogue(float v, const GemmParams& p,
                                               float* __restrict__ C,
                                               const float* __restrict__ aux,
                                               float* __restrict__ upd, int64_t off,
                                               int j) {
#pragma clang fp contract(off)
    switch (p.epilogue) {
        case EPI_BIAS:
            v = v + p.bias[j];
            break;
        case EPI_BIAS_RELU:
            v = fmaxf(0.0f, v + p.bias[j]);
            break;
        case EPI_RELU:
            v = fmaxf(0.0f, v);
            break;
        case EPI_RELU_GRAD:
            v = aux[off] > 0.0f ? v : 0.0f;
            break;
        case EPI_SGD: {
            const float step = p.lr * v;
            upd[off] = upd[off] - step;
            break;
        }
        default:
            break;
    }
    C[off] = v;
}

// The operand an epilogue reads besides the accumulator (bias[j], aux[off] or
// upd[off]), loaded before the K loop so its latency overlaps the MFMAs.
// One unconditional load through a pointer chosen by the (uniform)
// epilogue: a switch around several loads compiles to exec-masked branches
// that load into one register, and the compiler then waits for the first
// load before anything after it, the K loop's loads included.  Without an
// operand the load reads C[off] (off must be a valid element) and the value
// is not used.
__device__ __forceinline__ float epilogue_operand(const GemmParams& p,
                                                  const float* __restrict__ C,
                                                  const float* __restrict__ aux,
                                                  const float* __restrict__ upd, int64_t off,
                                                  int j) {
    const int e = p.epilogue;
    const float* src = (e == EPI_BIAS || e == EPI_BIAS_RELU) ? p.bias + j
                       : e == EPI_RELU_GRAD                  ? aux + off
                       : e == EPI_SGD                        ? upd + off
                                                             : C + off;
    return *src;
}

// store_epilogue with the extra operand already loaded (epilogue_operand).
__device__ __forceinline__ void store_epilogue_pre(float v, const GemmParams& p,
                                                   float* __restrict__ C,
                                                   float* __restrict__ upd, int64_t off,
                                                   float pre) {
#pragma clang fp contract(off)
    switch (p.epilogue) {
        case EPI_BIAS:
            v = v + pre;
            break;
        case EPI_BIAS_RELU:
            v = fmaxf(0.0f, v + pre);
            break;
        case EPI_RELU:
            v = fmaxf(0.0f, v);
            break;
        case EPI_RELU_GRAD:
            v = pre > 0.0f ? v : 0.0f;
            break;
        case EPI_SGD: {
            const float step = p.lr * v;
            upd[off] = pre - step;
            break;
        }
        default:
            break;
    }
    C[off] = v;
}

// store_epilogue_pre over a thread's N elements, with the epilogue switch
// taken once (switched per element, the compiler reloaded the kernel
// arguments before every element's store) and no wait between the stores
// (wait_vmem_idle: without it each element's stores waited for the previous
// element's, 0.8 us of the MLP step's weight-gradient GEMMs).
template <int E, int N>
__device__ __forceinline__ void store_epilogue_elems_as(const float (&v)[N],
                                                        const int64_t (&off)[N],
                                                        const bool (&live)[N],
                                                        const float (&pre)[N], float lr,
                                                        float* __restrict__ C,
                                                        float* __restrict__ upd) {
#pragma clang fp contract(off)
    float x[N], u[N];
#pragma unroll
    for (int q = 0; q < N; ++q) {
        x[q] = v[q];
        if (E == EPI_BIAS) x[q] = x[q] + pre[q];
        if (E == EPI_BIAS_RELU) x[q] = fmaxf(0.0f, x[q] + pre[q]);
        if (E == EPI_RELU) x[q] = fmaxf(0.0f, x[q]);
        if (E == EPI_RELU_GRAD) x[q] = pre[q] > 0.0f ? x[q] : 0.0f;
        if (E == EPI_SGD) {
            const float step = lr * x[q];
            u[q] = pre[q] - step;
        }
    }
    wait_vmem_idle();
#pragma unroll
    for (int q = 0; q < N; ++q) {
        if (!live[q]) continue;
        if (E == EPI_SGD) upd[off[q]] = u[q];
        C[off[q]] = x[q];
    }
}

template <int N>
__device__ __forceinline__ void store_epilogue_elems(const float (&v)[N], const int64_t (&off)[N],
                                                     const bool (&live)[N], const float (&pre)[N],
                                                     const GemmParams& p, float* __restrict__ C,
                                                     float* __restrict__ upd) {
    switch (p.epilogue) {
        case EPI_BIAS: store_epilogue_elems_as<EPI_BIAS>(v, off, live, pre, p.lr, C, upd); break;
        case EPI_BIAS_RELU:
            store_epilogue_elems_as<EPI_BIAS_RELU>(v, off, live, pre, p.lr, C, upd);
            break;
        case EPI_RELU: store_epilogue_elems_as<EPI_RELU>(v, off, live, pre, p.lr, C, upd); break;
        case EPI_RELU_GRAD:
            store_epilogue_elems_as<EPI_RELU_GRAD>(v, off, live, pre, p.lr, C, upd);
            break;
        case EPI_SGD: store_epilogue_elems_as<EPI_SGD>(v, off, live, pre, p.lr, C, upd); break;
        default: store_epilogue_elems_as<EPI_NONE>(v, off, live, pre, p.lr, C, upd); break;
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

// Epilogue of the LDS-tiled kernels: one wave's FM x FN block of 32x32
// accumulators, whose top-left element is C[mw][nw], goes through the
// epilogue into C.
//
// Interior wave blocks with an epilogue that reads nothing per element (none,
// bias, bias+ReLU, ReLU) take a fast path: stores through a buffer descriptor
// based at the block's corner, each lane's column and half-row as a 32-bit
// offset and the row part wave-uniform (a scalar offset), so a store costs no
// address arithmetic, no bounds test and no wait.  `bias_pre`, when given,
// holds this lane's bias value of each column block, fetched before the K
// loop.  The per-element path below it serves edge blocks and the epilogues
// that read aux or update a parameter.
constexpr int kBufferWord3Store = 0x00020000;  // raw-buffer descriptor word 3 (gfx9 family)

// STREAM = 1: the fast path's stores are non-temporal (buffer store `nt`), for
// tiles that only large outputs use (2048^3: 119.8 -> 118.6 us; 4096^3 and
// 8192^3 within 0.3%).
template <int FM, int FN, int STREAM = 0>
__device__ __forceinline__ void store_wave_tile(floatx16 (&acc)[FM][FN], const GemmParams& p,
                                                int64_t bz, int mw, int nw, int half,
                                                int l32, const float* bias_pre = nullptr) {
    {
        const int epi = p.epilogue;
        const bool plain = epi == EPI_NONE || epi == EPI_BIAS || epi == EPI_BIAS_RELU ||
                           epi == EPI_RELU;
        // Byte offsets stay below 2^31: (FM * 32 rows) * ldc * 4 bytes.
        if (plain && mw + FM * 32 <= p.M && nw + FN * 32 <= p.N &&
            p.ldc < (int64_t(1) << 29) / (FM * 32)) {
            const bool has_bias = epi == EPI_BIAS || epi == EPI_BIAS_RELU;
            const bool relu = epi == EPI_BIAS_RELU || epi == EPI_RELU;
            // mw and nw are wave-uniform by construction; saying so keeps the
            // descriptor in scalar registers.
            const int mwu = __builtin_amdgcn_readfirstlane(mw);
            const int nwu = __builtin_amdgcn_readfirstlane(nw);
            float* corner = p.C + bz * p.strideC + (int64_t)mwu * p.ldc + nwu;
            const __amdgpu_buffer_rsrc_t rsrc =
                __builtin_amdgcn_make_buffer_rsrc(corner, (short)0, -1, kBufferWord3Store);
            const int ldc = (int)p.ldc;
            const uint32_t lane_off = (uint32_t)((4 * half) * ldc + l32) * 4u;
            float bj[FN];
#pragma unroll
            for (int ni = 0; ni < FN; ++ni) {
                bj[ni] = has_bias ? (bias_pre ? bias_pre[ni] : p.bias[nw + ni * 32 + l32]) : 0.0f;
            }
            // One uniform branch on the epilogue, then straight-line stores.
            auto store_all = [&](auto op) __attribute__((always_inline)) {
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
#pragma unroll
                    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            const int row = mi * 32 + 8 * (r >> 2) + (r & 3);
                            const float v = op(acc[mi][ni][r], bj[ni]);
                            __builtin_amdgcn_raw_buffer_store_b32(
                                __builtin_bit_cast(uint32_t, v), rsrc, (int)lane_off,
                                (row * ldc + ni * 32) * 4, STREAM ? 2 : 0);  // 2: nt
                        }
            };
            if (has_bias && relu) {
                store_all([](float v, float b) { return fmaxf(0.0f, v + b); });
            } else if (has_bias) {
                store_all([](float v, float b) { return v + b; });
            } else if (relu) {
                store_all([](float v, float) { return fmaxf(0.0f, v); });
            } else {
                store_all([](float v, float) { return v; });
            }
            return;
        }
    }
    float* __restrict__ C = p.C + bz * p.strideC;
    const float* __restrict__ aux = p.aux ? p.aux + bz * p.strideC : nullptr;
    float* __restrict__ upd = p.upd ? p.upd + bz * p.strideC : nullptr;
    const int epi = p.epilogue;
    const bool has_bias = epi == EPI_BIAS || epi == EPI_BIAS_RELU;
    const bool relu = epi == EPI_BIAS_RELU || epi == EPI_RELU;
#pragma unroll
    for (int ni = 0; ni < FN; ++ni) {
        const int j = nw + ni * 32 + l32;
        const bool j_ok = j < p.N;
        // One bias value per lane and column block, loaded once.
        const float bj = (has_bias && j_ok) ? p.bias[j] : 0.0f;
#pragma unroll
        for (int mi = 0; mi < FM; ++mi) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = mw + mi * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (j_ok && i < p.M) {
                    const int64_t off = (int64_t)i * p.ldc + j;
                    float v = acc[mi][ni][r];
                    if (has_bias) v += bj;
                    if (relu) v = fmaxf(0.0f, v);
                    if (epi == EPI_RELU_GRAD) v = aux[off] > 0.0f ? v : 0.0f;
                    if (epi == EPI_SGD) {
#pragma clang fp contract(off)
                        const float step = p.lr * v;
                        upd[off] = upd[off] - step;
                    }
                    C[off] = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// LDS double-buffered MFMA tile kernel.  NT = 64 * (BM/WM) * (BN/WN) threads;
// each wave owns a WM x WN block of C made of (WM/32) x (WN/32) MFMA 32x32
// accumulators.  Per K-tile: the global loads of tile t+PF are issued first,
// the current LDS buffer feeds the MFMAs, then the registers holding tile t+1
// go to the other LDS buffer and one barrier closes the step.  With PF = 2
// two register sets alternate, so a tile's global loads have two K-tiles of
// MFMA work to land before the barrier needs them (with PF = 1 a late load
// stalls the whole block at the barrier).  PAD floats of padding per LDS row;
// WPE is the minimum number of waves per SIMD the register allocation must
// allow (occupancy target).
// ---------------------------------------------------------------------------
template <int BM_, int BN_, int BK_, int WM_, int WN_, int PAD_, int WPE_, int PRIO_ = 0,
          int KCH_ = BK_ / 2, int PF_ = 1, int PIPE_ = 0>
struct TileCfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int PAD = PAD_, WPE = WPE_, PRIO = PRIO_, KCH = KCH_, PF = PF_;
    static constexpr int PIPE = PIPE_;
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
        // Operand fragments are read from LDS a chunk of KCH k pairs at a
        // time, all before the chunk's first MFMA, so the LDS latency is paid
        // once per chunk rather than per k pair.  With PIPE the fragment
        // registers are double-buffered and the reads of chunk c+1 are issued
        // before the MFMAs of chunk c.
        constexpr int KP = BK / 2;
        constexpr int KCH = Cfg::KCH;
        constexpr int NCH = KP / KCH;
        static_assert(KP % KCH == 0, "chunk must divide the k pairs of a tile");
        static_assert(Cfg::PF == 1 || Cfg::PF == 2, "prefetch distance is 1 or 2 tiles");
        float a[2][KCH][FM];
        float b[2][KCH][FN];
        auto read_chunk = [&](const float* __restrict__ as, const float* __restrict__ bs, int c,
                              int slot) {
#pragma unroll
            for (int q = 0; q < KCH; ++q) {
                const int kk = 2 * (c * KCH + q) + half;
#pragma unroll
                for (int mi = 0; mi < FM; ++mi)
                    a[slot][q][mi] = as[kk * LoaderA::LD + wm0 + mi * 32 + l32];
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
                    b[slot][q][ni] = bs[kk * LoaderB::LD + wn0 + ni * 32 + l32];
            }
        };
        auto compute_tile = [&](const float* __restrict__ as, const float* __restrict__ bs) {
            if (Cfg::PIPE) read_chunk(as, bs, 0, 0);
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int slot = Cfg::PIPE ? (c & 1) : 0;
                if (Cfg::PIPE) {
                    if (c + 1 < NCH) read_chunk(as, bs, c + 1, slot ^ 1);
                } else {
                    read_chunk(as, bs, c, 0);
                }
                // Keep the scheduler from sinking the reads back next to their MFMAs.
                __builtin_amdgcn_sched_barrier(0);
                if (Cfg::PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
                for (int q = 0; q < KCH; ++q)
#pragma unroll
                    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                        for (int ni = 0; ni < FN; ++ni)
                            acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                a[slot][q][mi], b[slot][q][ni], acc[mi][ni], 0, 0, 0);
                if (Cfg::PRIO) __builtin_amdgcn_s_setprio(0);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        auto load_tile = [&](LoaderA& la, LoaderB& lb, int t) {
            const int k0 = t * BK;
            const bool chk = edge_mn || (k0 + BK > p.K);
            la.load(A, p.lda, p.M, p.K, m0, k0, tid, chk);
            lb.load(B, p.ldb, p.N, p.K, n0, k0, tid, chk);
        };

        LoaderA la0, la1;
        LoaderB lb0, lb1;
        load_tile(la0, lb0, 0);
        if (Cfg::PF == 2 && ktiles > 1) load_tile(la1, lb1, 1);
        la0.store(As[0], tid);
        lb0.store(Bs[0], tid);
        __syncthreads();

        if (Cfg::PF == 1) {
            for (int t = 0; t < ktiles; ++t) {
                const int cur = t & 1;
                const bool has_next = (t + 1) < ktiles;
                if (has_next) load_tile(la0, lb0, t + 1);
                compute_tile(As[cur], Bs[cur]);
                if (has_next) {
                    la0.store(As[cur ^ 1], tid);
                    lb0.store(Bs[cur ^ 1], tid);
                }
                __syncthreads();
            }
        } else {
            // Tile t's registers are set t & 1; the loop is unrolled by two so
            // both sets have fixed registers.  At step t the loads of tile t+2
            // go into the set that tile t left, and tile t+1's set, loaded one
            // step earlier, is written to LDS.
            auto step = [&](int t, LoaderA& la_next2, LoaderB& lb_next2, LoaderA& la_next1,
                            LoaderB& lb_next1) {
                const int cur = t & 1;
                if (t + 2 < ktiles) load_tile(la_next2, lb_next2, t + 2);
                compute_tile(As[cur], Bs[cur]);
                if (t + 1 < ktiles) {
                    la_next1.store(As[cur ^ 1], tid);
                    lb_next1.store(Bs[cur ^ 1], tid);
                }
                __syncthreads();
            };
            for (int t = 0; t < ktiles; t += 2) {
                step(t, la0, lb0, la1, lb1);
                if (t + 1 < ktiles) step(t + 1, la1, lb1, la0, lb0);
            }
        }
    }

    store_wave_tile<FM, FN>(acc, p, bz, m0 + wm0, n0 + wn0, half, l32);
}

// ---------------------------------------------------------------------------
// Direct-to-LDS tile kernel (gfx950 global_load_lds_dwordx4).
//
// Global memory is copied into LDS by the load unit itself: each 64-lane
// instruction moves 1 KB (16 bytes per lane, lane i to LDS base + 16 i) with
// no VGPR staging and no ds_write.  A ring of STAGES tile buffers keeps
// STAGES - 1 tiles of loads in flight; at K-tile t a wave waits until its own
// loads of tile t have landed (s_waitcnt vmcnt), then one s_barrier makes
// every wave's copy visible and releases the buffer of tile t - 1, which the
// loads of tile t + STAGES - 1 then refill.  The barrier is the raw
// s_barrier: the workgroup fence of __syncthreads would also wait for the
// loads still in flight for later tiles.
//
// Operand layouts in LDS, per stage:
//  * k-contiguous operand (A not transposed, B transposed): one row of BK = 16
//    floats per m (n), as four 16-byte k chunks whose order within the row is
//    permuted by kc_swz(row).  A lane reads its four k values of a chunk with
//    one ds_read_b128; the permutation spreads a wave's 32 rows over the LDS
//    banks.
//  * mn-contiguous operand (A transposed, B not transposed): one unpadded row
//    of MN floats per k, filled by whole 64-lane copies (measured
//    conflict-free for the ds_read_b32 of two half-waves on rows 4 apart).
//
// MFMA k order: within each group of 8 reduction steps, MFMA q (q = 0..3)
// takes k = 8g + q from lanes 0-31 and k = 8g + 4 + q from lanes 32-63, the
// same permutation for both operands, so every k is summed exactly once and
// a lane's four A (or B) values of a group are one contiguous chunk.
//
// Host contract: K is a multiple of 4 (the last K-tile may be partial) and
// the operands satisfy the 16-byte vector conditions (base, ld and batch
// stride multiples of 4 floats; an mn-contiguous operand's extent a multiple
// of 4).  Rows (columns) past M (N) are clamped to the last valid one: they
// only feed accumulators that are never stored.
// ---------------------------------------------------------------------------
// KS > 1 splits each K-tile's k-groups over KS sets of waves that share the
// block's LDS stages (more waves per SIMD for the same tile); their partial
// sums are added in set order after the K loop.
// CW is the copy width in floats per lane (4: 16-byte copies, which need
// 16-byte-aligned operand rows and K % 4 == 0; 1: 4-byte copies, any shape).
// ASM = 1: the steady-state K loop is a hand-scheduled one of dma_loops.inc
// (CfgDma256W4 and CfgDma128W4, every layout; see its generator).
template <int BM_, int BN_, int BK_, int WM_, int WN_, int STAGES_, int XPIPE_ = 0,
          int ILV_ = 0, int KS_ = 1, int CW_ = 4, int WPE_ = 1, int ASM_ = 0>
struct DmaCfg {
    static constexpr int ASM = ASM_;
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int STAGES = STAGES_;
    static constexpr int XPIPE = XPIPE_, ILV = ILV_, KS = KS_, CW = CW_;
    static constexpr int WPE = WPE_;  // waves per SIMD the register budget must allow
    static constexpr int NT = kWave * (BM / WM) * (BN / WN) * KS;
};

// s_waitcnt immediate: wait until at most n vector-memory operations of this
// wave are outstanding (lgkmcnt and expcnt unconstrained).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// One 16-byte-per-lane global -> LDS copy (lane i writes lds + 4 i floats;
// `lds` must be wave-uniform).  Kept out of the kernel templates so that the
// host pass, which cannot type-check this device builtin, never sees it.
__device__ __forceinline__ void dma_copy16(const float* g, float* lds) {
    __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

// The same with 4 bytes per lane (lane i writes lds + i floats).
__device__ __forceinline__ void dma_copy4(const float* g, float* lds) {
    __builtin_amdgcn_global_load_lds(g, lds, 4, 0, 0);
}

// 4-byte copies through a buffer descriptor: `base` is wave-uniform (scalar
// registers) and each lane adds its own 32-bit byte offset, so a copy costs
// one VGPR instead of a 64-bit address.  Descriptor word 3 is the raw-buffer
// value for gfx9-family targets (gfx950 included).
constexpr int kBufferWord3 = 0x00020000;

// A pointer the caller knows to be the same on every lane, in scalar
// registers: without this the compiler may treat a descriptor built from it
// as divergent and wrap each buffer load in a loop over the lanes' values.
__device__ __forceinline__ const float* wave_uniform(const float* q) {
    const uint64_t v = (uint64_t)q;
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const float*)(lo | (hi << 32));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dma_buffer(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, -1, kBufferWord3);
}

// The same with 16 bytes per lane (lane i writes lds + 4 i floats).
__device__ __forceinline__ void dma_buf_copy16(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_off,
                                               float* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds, 16, byte_off, 0, 0, 0);
}

__device__ __forceinline__ void dma_buf_copy4(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_off,
                                              float* lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds, 4, byte_off, 0, 0, 0);
}

// Chunk permutation of a k-contiguous LDS row of CPR 16-byte chunks.  Both
// forms were measured conflict-free with the LDS bank-conflict counter on
// gfx950 for a ds_read_b128 of 32 consecutive rows x one chunk (4 chunks per
// row: rows 4j .. 4j+3 rotate by j; without a permutation the read costs 37%
// extra LDS cycles, and with ((r >> 1) ^ (r >> 3)) & 3 it costs 17%).
template <int CPR>
__device__ __forceinline__ int kc_swz(int r) {
    static_assert(CPR == 4 || CPR == 8 || CPR == 16, "4, 8 or 16 chunks per row");
    if (CPR == 4) return (r >> 2) & 3;
    if (CPR == 8) return (r ^ (r >> 3)) & 7;
    return r & 15;  // 16 chunks: measured conflict-free, (r >> 1) & 15 costs 10%
}

// Chunk rotation of a k-contiguous tile of 16-float rows read by 16x16x4
// MFMA fragments (lane l: row l % 16, chunk l / 16, one ds_read_b128).  A
// ds_read_b128 is served in four passes of 16 lanes, lane l in the pass of
// (l / 32, parity of bits 2..4 of l), each free of bank conflicts when its
// lanes' 16-byte slots differ mod 16 (measured with the LDS bank-conflict
// counter).  kc_swz<4>, right for the 32x32 fragments' lanes (32 rows x one
// chunk), gives these lanes two-way conflicts; swapping the chunks of rows
// 4..7 and 12..15 in pairs (XOR 2) gives none.
__device__ __forceinline__ int kc_swz16(int r) { return (r >> 1) & 2; }

// One global -> LDS copy operand.  CW is the copy width in floats per lane:
// 4 (16-byte copies; needs 16-byte-aligned rows) or 1 (4-byte copies; any
// alignment, any K).  Either way the LDS image is the same, so the fragment
// reads are shared: a k-contiguous operand is stored as rows of BK floats
// whose 16-byte chunks are rotated by kc_swz, an mn-contiguous operand as
// unpadded rows of MN floats.  With CW = 1 a copy's 64 lanes fill 64
// consecutive LDS floats, each lane fetching the global element that belongs
// there, so one copy still reads one contiguous row segment.
template <int MN, int BK, int NT, bool KC, int CW = 4>
struct DmaOperand {
    static constexpr int CPR = BK / 4;                     // k chunks per k-contiguous row
    static constexpr int LDR = KC ? BK : MN;               // floats per LDS row
    static constexpr int STAGE = MN * BK;                  // floats per stage
    static constexpr int UNITS = MN * BK / CW;             // copy units per stage
    static constexpr int INS = UNITS / kWave;              // 64-lane copies per stage
    // Copies per lane per tile.  When the stage's copies do not divide evenly
    // over the block's waves, every wave still issues PER of them and the
    // surplus ones repeat the stage's last copy (the same bytes to the same
    // LDS place), so each wave's count of copies in flight, which the
    // kernel's vmcnt waits rely on, is the same.
    static constexpr int PER = (UNITS + NT - 1) / NT;
    __device__ __forceinline__ static int ins_of(int wave, int i) {
        return min(wave * PER + i, INS - 1);
    }
    static_assert(CW == 4 || CW == 1, "16- or 4-byte copies");
    static_assert(UNITS % kWave == 0, "a stage is whole 64-lane copies");
    static_assert(!KC || CPR == 4 || CPR == 8 || CPR == 16,
                  "BK of 16, 32 or 64 for a k-contiguous operand");
    static_assert(!KC || (kWave * CW) % BK == 0, "a copy covers whole k-contiguous rows");
    static_assert(CW == 4 || !KC || BK == kWave, "4-byte copies of k-contiguous rows: BK = 64");
    // With 16-byte copies a lane's chunk must not straddle two rows; with
    // 4-byte copies each lane places its own element, so a copy may.
    static_assert(CW == 1 || KC || (kWave * CW) % MN == 0 || MN % (kWave * CW) == 0,
                  "mn-contiguous rows must tile the 64-lane copies");
    // Global offset of each copy at k0 = 0: the wave's base (gb0, the row of
    // its first copy; wave-uniform, so in scalar registers) plus a 32-bit
    // lane part per copy (lo), one VGPR per copy.  The copies are buffer
    // loads from a descriptor at the wave's base, so no copy needs a 64-bit
    // address.  The lane part spans the wave's copies' rows (at most 64):
    // callers keep leading dimensions below kDmaMaxLd.
    int64_t gb0;
    int lo[PER];
    int loff[PER];      // wave-uniform LDS offset (floats) of each copy within a stage

    // Position (in the tile) of copy unit `slot`: the operand row or k row
    // `r`, and the offset along the contiguous dimension `c`.
    __device__ __forceinline__ static void place(int slot, int& r, int& c) {
        const int f = slot * CW;  // LDS float offset within the stage
        if (KC) {
            r = f / BK;
            const int p = f % BK;
            c = 4 * ((p / 4) ^ kc_swz<CPR>(r)) + p % 4;  // global k within the tile
        } else {
            r = f / MN;  // k row
            c = f % MN;  // column
        }
    }

    __device__ __forceinline__ void init(int64_t ld, int mn0, int mn_lim, int tid) {
        const int lane = tid & (kWave - 1);
        // Wave-uniform by construction; readfirstlane lets the compiler keep
        // loff in scalar registers, so each copy sets M0 without a VALU step.
        const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
        // Row of the wave's first copy (the same for every lane).
        int r0, c0;
        place(ins_of(wave, 0) * kWave, r0, c0);
        const int row0 = KC ? min(mn0 + r0, mn_lim - 1) : r0;
        gb0 = (int64_t)row0 * ld;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int ins = ins_of(wave, i);
            int r, c;
            place(ins * kWave + lane, r, c);
            if (KC) {
                lo[i] = (int)((int64_t)(min(mn0 + r, mn_lim - 1) - row0) * ld) + c;
            } else {
                lo[i] = (int)((int64_t)(r - row0) * ld) + min(mn0 + c, mn_lim - CW);
            }
            loff[i] = ins * kWave * CW;
        }
    }

    // Copies the tile whose first reduction index is k0 into `stage`.  In
    // the tile that crosses K the copies past K are redirected to the last
    // valid element or row (with CW = 4, K is a multiple of 4, so a chunk is
    // either wholly inside or wholly past K): the kernel zeroes the fragment
    // values read from those slots, so they never count.
    __device__ __forceinline__ void issue(const float* __restrict__ base, int64_t ld, int k0,
                                          int K, float* stage, int tid) const {
        if (k0 + BK <= K) {
            issue_full(base, ld, k0, stage);
        } else {
            issue_tail(base, ld, k0, K, stage, tid);
        }
    }

    __device__ __forceinline__ static void copy(const float* g, float* lds) {
        if (CW == 4) {
            dma_copy16(g, lds);
        } else {
            dma_copy4(g, lds);
        }
    }

    // A tile wholly inside K: no per-copy bounds work.
    __device__ __forceinline__ void issue_full(const float* __restrict__ base, int64_t ld, int k0,
                                               float* stage) const {
        issue_part<0, PER>(base, ld, k0, stage);
    }

    // Copies I0 .. I1-1 of issue_full (a tile may be copied in parts).
    template <int I0, int I1>
    __device__ __forceinline__ void issue_part(const float* __restrict__ base, int64_t ld, int k0,
                                               float* stage) const {
        static_assert(0 <= I0 && I0 <= I1 && I1 <= PER, "a range of this tile's copies");
        if constexpr (I0 < I1) {
            const int64_t koff = KC ? (int64_t)k0 : (int64_t)k0 * ld;
            // The tile's wave-uniform base in a buffer descriptor (scalar
            // registers), each copy's lane part as a 32-bit offset from it.
            // (4096^3 from global_load_lds with 64-bit addresses: 909.5 ->
            // 905.8 us; 1024^3 20.8 -> 19.5 us; 1536^3 79.7 -> 72.9 us.)
            const __amdgpu_buffer_rsrc_t rsrc = dma_buffer(wave_uniform(base + (gb0 + koff)));
#pragma unroll
            for (int i = I0; i < I1; ++i) {
                if constexpr (CW == 4) {
                    dma_buf_copy16(rsrc, (uint32_t)lo[i] * 4u, stage + loff[i]);
                } else {
                    dma_buf_copy4(rsrc, (uint32_t)lo[i] * 4u, stage + loff[i]);
                }
            }
        }
    }

    __device__ __forceinline__ void issue_tail(const float* __restrict__ base, int64_t ld, int k0,
                                               int K, float* stage, int tid) const {
        const int lane = tid & (kWave - 1);
        const int wave = tid / kWave;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            int r, c;
            place(ins_of(wave, i) * kWave + lane, r, c);
            const int64_t g = gb0 + lo[i];
            int64_t off;
            if (KC) {
                off = g - c + min(k0 + c, K - CW);
            } else {
                off = g + (int64_t)(min(k0 + r, K - 1) - r) * ld;
            }
            copy(base + off, stage + loff[i]);
        }
    }

    // Operand values of MFMA q of group g for fragment row/col `idx` (the
    // wave's offset plus l32): v[q].
    __device__ __forceinline__ void read(const float* stage, int g, int idx, int half,
                                         float v[4]) const {
        if (KC) {
            const int pos = (2 * g + half) ^ kc_swz<CPR>(idx);
            const floatx4 x = *reinterpret_cast<const floatx4*>(stage + idx * LDR + 4 * pos);
            v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = stage[(8 * g + 4 * half + q) * LDR + idx];
        }
    }
};

// f(std::integral_constant<int, 0>{}) .. f(std::integral_constant<int, N - 1>{}).
template <class F, int... G>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, G...>) {
    (f(std::integral_constant<int, G>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Scheduling hint for one MFMA group: after MFMA j, the reads and copies
// that bring the running totals to ceil(total * (j + 1) / kMfma), so both are
// spread evenly over the group (the builtin needs constant counts).
template <int kMfma, int kReads, int kCopies, int J>
__device__ __forceinline__ void spread_hint_one() {
    constexpr int r = (kReads * (J + 1) + kMfma - 1) / kMfma - (kReads * J + kMfma - 1) / kMfma;
    constexpr int c = (kCopies * (J + 1) + kMfma - 1) / kMfma - (kCopies * J + kMfma - 1) / kMfma;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);  // DS reads
    if constexpr (c > 0) __builtin_amdgcn_sched_group_barrier(0x010, c, 0);  // VMEM
}

template <int kMfma, int kReads, int kCopies, int... J>
__device__ __forceinline__ void spread_hint(std::integer_sequence<int, J...>) {
    (spread_hint_one<kMfma, kReads, kCopies, J>(), ...);
}

// The same for a group whose fragment reads come before its copies in
// program order (the copies write LDS, so the compiler keeps every read
// ahead of them): the reads spread over the first kSpan MFMAs, the copies
// over the rest.
template <int kMfma, int kReads, int kCopies, int kSpan, int J>
__device__ __forceinline__ void front_hint_one() {
    static_assert(kSpan > 0 && kSpan < kMfma, "reads and copies each get some MFMAs");
    constexpr int M2 = kMfma - kSpan, J2 = J - kSpan;
    constexpr int r = J < kSpan ? (kReads * (J + 1) + kSpan - 1) / kSpan - (kReads * J + kSpan - 1) / kSpan : 0;
    constexpr int c = J >= kSpan ? (kCopies * (J2 + 1) + M2 - 1) / M2 - (kCopies * J2 + M2 - 1) / M2 : 0;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);  // DS reads
    if constexpr (c > 0) __builtin_amdgcn_sched_group_barrier(0x010, c, 0);  // VMEM
}

template <int kMfma, int kReads, int kCopies, int kSpan, int... J>
__device__ __forceinline__ void front_hint(std::integer_sequence<int, J...>) {
    (front_hint_one<kMfma, kReads, kCopies, kSpan, J>(), ...);
}

// Block -> (batch, tile) for a launch whose 1-D grid covers every tile of
// every batch (few tiles per batch): renumbered so each XCD owns one
// contiguous range of (batch, tile) pairs, i.e. whole batches when the batch
// count is a multiple of 8.  A batch's tiles share its operand panels, which
// then come into one XCD's L2 once.
__device__ __forceinline__ void flat_batch_coords(int bid, int nblocks, int tiles_m, int tiles_n,
                                                  int& tm, int& tn, int64_t& bz) {
    if ((nblocks & 7) == 0) bid = (bid & 7) * (nblocks >> 3) + (bid >> 3);
    const int tiles = tiles_m * tiles_n;
    bz = bid / tiles;
    const int t = bid - (int)bz * tiles;
    tm = t % tiles_m;
    tn = t / tiles_m;
}

// The operands' addresses, batch strides, leading dimensions and shape, the
// bias and the epilogue kind come as leading scalar arguments, which arrive
// preloaded in SGPRs (14 dwords; the compiler preloads only leading
// arguments that are not aggregates): the bias load and the first copies
// then wait for no scalar load of the GemmParams aggregate, which supplies
// only what the epilogue needs.  `mode` holds the epilogue kind in its low 8
// bits and, for a 1-D grid over every tile of every batch (few tiles per
// batch, see flat_batch_coords), the batch count above them (0: grid.y is
// the batch and grid.x the tiles).
template <class Cfg, bool TA, bool TB>
__global__ void __launch_bounds__(Cfg::NT, Cfg::WPE)
sgemm_dma_kernel(const float* __restrict__ A0, const float* __restrict__ B0,
                 const float* __restrict__ bias, int strideA, int strideB, int lda, int ldb, int M,
                 int N, int K, int mode, GemmParams pa) {
    GemmParams p = pa;
    p.A = A0;
    p.B = B0;
    p.bias = bias;
    p.strideA = strideA;
    p.strideB = strideB;
    p.lda = lda;
    p.ldb = ldb;
    p.M = M;
    p.N = N;
    p.K = K;
    p.epilogue = mode & 255;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, WM = Cfg::WM, WN = Cfg::WN;
    constexpr int NT = Cfg::NT, S = Cfg::STAGES;
    constexpr int FM = WM / 32, FN = WN / 32, WGM = BM / WM;
    constexpr int NG = BK / 8;
    constexpr int KS = Cfg::KS;
    constexpr int WMN = (BM / WM) * (BN / WN);  // waves of one k-group set
    constexpr int NGK = NG / KS;                // k-groups per tile for each set
    static_assert(NG % KS == 0, "the k-groups of a tile divide evenly over the sets");
    static_assert(KS == 1 || Cfg::XPIPE != 0, "k-group sets need the cross-tile pipeline");
    using OpA = DmaOperand<BM, BK, NT, !TA, Cfg::CW>;
    using OpB = DmaOperand<BN, BK, NT, TB, Cfg::CW>;
    constexpr int PER_TILE = OpA::PER + OpB::PER;
    static_assert(S >= 2 && S <= 4, "2 to 4 stages");
    static_assert((S - 1) * PER_TILE <= 63, "copies in flight fit the 6-bit vmcnt counter");
    __shared__ __attribute__((aligned(16))) float lds[S * (OpA::STAGE + OpB::STAGE)];
    float* const As = lds;
    float* const Bs = lds + S * OpA::STAGE;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int l32 = lane & 31;
    const int half = lane >> 5;
    const int kset = wave / WMN;                // which k-group set
    const int wmn = wave % WMN;
    const int wm0 = (wmn % WGM) * WM;
    const int wn0 = (wmn / WGM) * WN;
    const int g0 = kset * NGK;                  // this set's first k-group of a tile

    // (the tile counts and the grid's size follow from the shape: gridDim.x
    // would be a scalar load from the dispatch's implicit arguments)
    const int tiles_m = (M + BM - 1) / BM;
    const int tiles_n = (N + BN - 1) / BN;
    const int flat_batches = mode >> 8;
    int tm, tn;
    int64_t bz;
    if (flat_batches) {
        flat_batch_coords(blockIdx.x, tiles_m * tiles_n * flat_batches, tiles_m, tiles_n, tm, tn,
                          bz);
    } else {
        tile_coords(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, tm, tn);
        bz = blockIdx.y;
    }
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const float* __restrict__ A = p.A + bz * p.strideA;
    const float* __restrict__ B = p.B + bz * p.strideB;

    OpA opa;
    OpB opb;
    opa.init(p.lda, m0, p.M, tid);
    opb.init(p.ldb, n0, p.N, tid);

    floatx16 acc[FM][FN];
#pragma unroll
    for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int ni = 0; ni < FN; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;

    // This lane's bias value of each column block, for the epilogue.  Issued
    // before the first copies, so the explicit vmcnt counts of the copies below
    // (which count only later operations) stay exact.
    float bias_pre[FN];
    if (p.epilogue == EPI_BIAS || p.epilogue == EPI_BIAS_RELU) {
#pragma unroll
        for (int ni = 0; ni < FN; ++ni) bias_pre[ni] = p.bias[min(n0 + wn0 + ni * 32 + l32, p.N - 1)];
    } else {
#pragma unroll
        for (int ni = 0; ni < FN; ++ni) bias_pre[ni] = 0.0f;
    }

    // K need only be a multiple of 4: the last K-tile may be partial.
    const int ktiles = (p.K + BK - 1) / BK;
    const int tail_tile = (p.K % BK) ? ktiles - 1 : -1;
    auto issue_tile = [&](int t, int s) {
        opa.issue(A, p.lda, t * BK, p.K, As + s * OpA::STAGE, tid);
        opb.issue(B, p.ldb, t * BK, p.K, Bs + s * OpB::STAGE, tid);
    };
    // A K range of at most S tiles is copied whole up front, each tile into
    // its own stage (the pipelined loop issues only S - 1 ahead and the last
    // tile after the first has landed).  The cross-tile pipeline keeps its
    // own schedule.
    const bool all_ahead = !Cfg::XPIPE && ktiles <= S;
#pragma unroll
    for (int s = 0; s < S - 1; ++s) {
        if (s < ktiles) issue_tile(s, s);
    }
    if (all_ahead && ktiles == S) issue_tile(S - 1, S - 1);

    float a[2][4][FM];
    float b[2][4][FN];
    // Reads group g of tile `tile` into register slot `slot`.  `masked` (a
    // compile-time flag, so the steady-state loop has no branch between the
    // reads and the MFMAs) marks the tile that crosses K: there A and B
    // values at k >= K are zeroed (the LDS slots past K hold redirected copies
    // of valid data; zeroing both keeps an infinity there from turning into
    // 0 * inf).
    auto read_group = [&](const float* as, const float* bs, int g, int slot, int tile,
                          auto masked) __attribute__((always_inline)) {
        float v[4];
#pragma unroll
        for (int mi = 0; mi < FM; ++mi) {
            opa.read(as, g, wm0 + mi * 32 + l32, half, v);
#pragma unroll
            for (int q = 0; q < 4; ++q) a[slot][q][mi] = v[q];
        }
#pragma unroll
        for (int ni = 0; ni < FN; ++ni) {
            opb.read(bs, g, wn0 + ni * 32 + l32, half, v);
#pragma unroll
            for (int q = 0; q < 4; ++q) b[slot][q][ni] = v[q];
        }
        if constexpr (decltype(masked)::value) {
            const int kbase = tile * BK + 8 * g + 4 * half;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
                for (int mi = 0; mi < FM; ++mi)
                    a[slot][q][mi] = kbase + q < p.K ? a[slot][q][mi] : 0.0f;
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
                    b[slot][q][ni] = kbase + q < p.K ? b[slot][q][ni] : 0.0f;
            }
        }
    };

    auto mfma_group = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                        a[slot][q][mi], b[slot][q][ni], acc[mi][ni], 0, 0, 0);
    };
    // The fragment reads the hints below spread: FM b128 A reads and about
    // two instructions per B fragment.  One more for the one-column-fragment
    // tiles of the 128-row and 4-byte-copy configs (measured, warmed clock:
    // 2048^3 130.2 -> 128.5 us, 1023^3 24.0 -> 23.4 us; the same at the
    // 16-byte 64x64 tile made 1000^3 and 1024^3 1-2% slower).
    constexpr int kHintReads = FM + 2 * FN + ((FN == 1 && (BM == 128 || Cfg::CW == 1)) ? 1 : 0);
    // With ILV the scheduler is asked to spread the LDS reads of the next
    // group between this group's MFMAs (two MFMAs, one read, ...).
    auto interleave_hint = [&]() {
        if (Cfg::ILV) {
            constexpr int kReads = kHintReads;
            constexpr int kMfma = 4 * FM * FN;
            constexpr int kPer = kMfma >= 2 * kReads ? 2 : 1;
            constexpr int kPairs = kMfma / kPer < kReads ? kMfma / kPer : kReads;
#pragma unroll
            for (int j = 0; j < kPairs; ++j) {
                __builtin_amdgcn_sched_group_barrier(0x008, kPer, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            if (kMfma > kPer * kPairs)
                __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kPer * kPairs, 0);
        }
    };
    // The same for the group that also issues the next tile's copies: after
    // each MFMA, an even share of the fragment reads (DS) and copies (VMEM).
    auto interleave_hint_copies = [&]() {
        if (Cfg::ILV) {
            constexpr int kMfma = 4 * FM * FN;
            spread_hint<kMfma, kHintReads, PER_TILE>(std::make_integer_sequence<int, kMfma>{});
        }
    };

    if constexpr (Cfg::XPIPE != 0) {
        // Cross-tile pipeline: the barrier sits before the last group's
        // MFMAs, so the first reads of tile t+1 are in flight while those
        // MFMAs run.  The last group's fragments are read before the barrier,
        // so at the barrier every wave has read all of tile t (lgkmcnt 0) and
        // tile t+1 has landed.
        // S = 2: tile t's stage is then free, and tile t+2 goes into it in
        // the group after the barrier (the copies share that group's MFMAs).
        // S = 3: tile t+2 goes into tile t-1's stage, free since the previous
        // barrier, so its copies are spread over all of tile t's groups
        // (chunk g in group g).  The barrier then waits for tile t+1 only,
        // with the chunks of tile t+2 issued before it still in flight.
        static_assert((S == 2 || S == 3) && NGK % 2 == 0,
                      "cross-tile pipeline: 2 or 3 stages, even group count");
        using No = std::false_type;
        using Yes = std::true_type;
        // Copies of chunk g of a tile: [chunk_lo(g), chunk_lo(g + 1)) of the
        // tile's PER_TILE copies (A's, then B's).
        constexpr auto chunk_lo = [](int g) { return g * PER_TILE / NGK; };
        constexpr int kPre = S == 3 ? chunk_lo(NGK - 1) : 0;  // copies issued before the barrier
        const bool has_tail = tail_tile >= 0;
        // Tiles 0 .. S-2 are in flight; with S = 2 add tile 1; wait for tile 0.
        if (S == 2 && ktiles > 1) issue_tile(1, 1);
        if (ktiles > 1) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER_TILE));
        } else {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        int t = 0;  // the next K-tile the C++ loops below run
        if constexpr (Cfg::ASM != 0) {
            static_assert(S == 3 && KS == 1 && Cfg::CW == 4 && NT == 256 &&
                              ((BM == 256 && BN == 256 && BK == 16 && FM == 4 && FN == 4) ||
                               (BM == 128 && BN == 128 && BK == 32 && FM == 2 && FN == 2) ||
                               (BM == 64 && BN == 64 && BK == 64 && FM == 1 && FN == 1)),
                          "the hand-scheduled loops are written for CfgDma256W4, CfgDma128W4 "
                          "and CfgDma64W4");
            static_assert(OpA::PER == 4 && OpB::PER == 4, "four copies of each operand per wave");
            // Whole groups of three steady K-tiles (tile t+2 full and inside
            // K) run in the asm loop; it starts where this code stands (tiles
            // 0 and 1 issued, tile 0 landed) and leaves the C++ loops the same
            // state at tile 3 * cnt, stage 0: group 0 of that tile is read
            // again below, tile 3 * cnt + 1 is in flight.
            int cnt = (has_tail ? ktiles - 3 : ktiles - 2) / 3;
            if (cnt > 0) {
                t = 3 * cnt;
                // Copies: each operand's base in a buffer descriptor, the lane
                // offsets of the wave's four copies, the K-tile's offset in a
                // scalar (tile 2 first); the host keeps every offset below 2^31.
                const __amdgpu_buffer_rsrc_t rsa = dma_buffer(wave_uniform(A));
                const __amdgpu_buffer_rsrc_t rsb = dma_buffer(wave_uniform(B));
                auto full = [](int64_t gb, int lane_part) { return (uint32_t)((gb + lane_part) * 4); };
                const uint32_t va0 = full(opa.gb0, opa.lo[0]), va1 = full(opa.gb0, opa.lo[1]),
                               va2 = full(opa.gb0, opa.lo[2]), va3 = full(opa.gb0, opa.lo[3]);
                const uint32_t vb0 = full(opb.gb0, opb.lo[0]), vb1 = full(opb.gb0, opb.lo[1]),
                               vb2 = full(opb.gb0, opb.lo[2]), vb3 = full(opb.gb0, opb.lo[3]);
                // one K-tile of each operand in bytes: BK floats along a
                // k-contiguous row, BK rows of an mn-contiguous operand
                const uint32_t astep = __builtin_amdgcn_readfirstlane(
                    (uint32_t)(TA ? BK * p.lda * 4 : BK * 4));
                const uint32_t bstep = __builtin_amdgcn_readfirstlane(
                    (uint32_t)(TB ? BK * 4 : BK * p.ldb * 4));
                uint32_t soa = 2 * astep;
                uint32_t sob = 2 * bstep;
                // LDS byte addresses: each copy's wave base (M0, before the
                // stage offset) and the lanes' fragment read bases.
                const uint32_t lds_a = (uint32_t)(uintptr_t)As;
                const uint32_t lds_b = (uint32_t)(uintptr_t)Bs;
                const uint32_t ma0 = __builtin_amdgcn_readfirstlane(lds_a + opa.loff[0] * 4);
                const uint32_t ma1 = __builtin_amdgcn_readfirstlane(lds_a + opa.loff[1] * 4);
                const uint32_t ma2 = __builtin_amdgcn_readfirstlane(lds_a + opa.loff[2] * 4);
                const uint32_t ma3 = __builtin_amdgcn_readfirstlane(lds_a + opa.loff[3] * 4);
                const uint32_t mb0 = __builtin_amdgcn_readfirstlane(lds_b + opb.loff[0] * 4);
                const uint32_t mb1 = __builtin_amdgcn_readfirstlane(lds_b + opb.loff[1] * 4);
                const uint32_t mb2 = __builtin_amdgcn_readfirstlane(lds_b + opb.loff[2] * 4);
                const uint32_t mb3 = __builtin_amdgcn_readfirstlane(lds_b + opb.loff[3] * 4);
                // Fragment read bases, as DmaOperand::read.  A k-contiguous
                // operand: row r's 16-byte k-chunk (2g + half) rotated by
                // kc_swz(r), per k-group and block (rka, rkb).  An
                // mn-contiguous one: the lane's column at k row 4 * half, per
                // block (rma, rmb).  Each loop reads the ones its layout has.
                uint32_t rka[NGK][FM], rkb[NGK][FN], rma[FM], rmb[FN];
#pragma unroll
                for (int g = 0; g < NGK; ++g) {
#pragma unroll
                    for (int mi = 0; mi < FM; ++mi) {
                        const int r = wm0 + mi * 32 + l32;
                        rka[g][mi] = lds_a + r * BK * 4 + 16 * ((2 * g + half) ^ kc_swz<OpA::CPR>(r));
                    }
#pragma unroll
                    for (int ni = 0; ni < FN; ++ni) {
                        const int r = wn0 + ni * 32 + l32;
                        rkb[g][ni] = lds_b + r * BK * 4 + 16 * ((2 * g + half) ^ kc_swz<OpB::CPR>(r));
                    }
                }
#pragma unroll
                for (int mi = 0; mi < FM; ++mi) rma[mi] = lds_a + (4 * half * BM + wm0 + mi * 32 + l32) * 4;
#pragma unroll
                for (int ni = 0; ni < FN; ++ni) rmb[ni] = lds_b + (4 * half * BN + wn0 + ni * 32 + l32) * 4;
                int m0s;
#define FDL_W4_LOOP(NAME)                                                                 \
    asm volatile(NAME##_TEXT                                                              \
                 : NAME##_ACC, [cnt] "+s"(cnt), [m0s] "=&s"(m0s), [soa] "+s"(soa),       \
                   [sob] "+s"(sob)                                                        \
                 : [ma0] "s"(ma0), [ma1] "s"(ma1), [ma2] "s"(ma2), [ma3] "s"(ma3),        \
                   [mb0] "s"(mb0), [mb1] "s"(mb1), [mb2] "s"(mb2), [mb3] "s"(mb3),        \
                   [astep] "s"(astep), [bstep] "s"(bstep), [rsa] "s"(rsa), [rsb] "s"(rsb), \
                   [va0] "v"(va0), [va1] "v"(va1), [va2] "v"(va2), [va3] "v"(va3),        \
                   [vb0] "v"(vb0), [vb1] "v"(vb1), [vb2] "v"(vb2), [vb3] "v"(vb3),        \
                   NAME##_READS                                                           \
                 : "v160", "v161", "v162", "v163", "v164", "v165", "v166", "v167",        \
                   "v168", "v169", "v170", "v171", "v172", "v173", "v174", "v175",        \
                   "v176", "v177", "v178", "v179", "v180", "v181", "v182", "v183",        \
                   "v184", "v185", "v186", "v187", "v188", "v189", "v190", "v191",        \
                   "v192", "v193", "v194", "v195", "v196", "v197", "v198", "v199",        \
                   "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207",        \
                   "v208", "v209", "v210", "v211", "v212", "v213", "v214", "v215",        \
                   "v216", "v217", "v218", "v219", "v220", "v221", "v222", "v223", "scc", \
                   "memory")
                if constexpr (BM == 256) {
                    if constexpr (!TA && !TB) {
                        FDL_W4_LOOP(FDL_DMA256W4_NN);
                    } else if constexpr (!TA) {
                        FDL_W4_LOOP(FDL_DMA256W4_NT);
                    } else if constexpr (!TB) {
                        FDL_W4_LOOP(FDL_DMA256W4_TN);
                    } else {
                        FDL_W4_LOOP(FDL_DMA256W4_TT);
                    }
                } else if constexpr (BM == 128) {
                    if constexpr (!TA && !TB) {
                        FDL_W4_LOOP(FDL_DMA128W4_NN);
                    } else if constexpr (!TA) {
                        FDL_W4_LOOP(FDL_DMA128W4_NT);
                    } else if constexpr (!TB) {
                        FDL_W4_LOOP(FDL_DMA128W4_TN);
                    } else {
                        FDL_W4_LOOP(FDL_DMA128W4_TT);
                    }
                } else {
                    if constexpr (!TA && !TB) {
                        FDL_W4_LOOP(FDL_DMA64W4_NN);
                    } else if constexpr (!TA) {
                        FDL_W4_LOOP(FDL_DMA64W4_NT);
                    } else if constexpr (!TB) {
                        FDL_W4_LOOP(FDL_DMA64W4_TN);
                    } else {
                        FDL_W4_LOOP(FDL_DMA64W4_TT);
                    }
                }
#undef FDL_W4_LOOP
            }
        }
        // Group 0 of tile t (stage 0: t is 0 or a multiple of 3).
        if (tail_tile == t) {
            read_group(As, Bs, g0, 0, t, Yes{});
        } else {
            read_group(As, Bs, g0, 0, t, No{});
        }
        // Stage of tile t is t % S; `cur` carries it (no division in the loop).
        auto next_stage = [](int c) { return c + 1 == S ? 0 : c + 1; };
        auto copy_chunk = [&](auto gc, int k0, int dst) __attribute__((always_inline)) {
            constexpr int c0 = chunk_lo(decltype(gc)::value);
            constexpr int c1 = chunk_lo(decltype(gc)::value + 1);
            constexpr int PA = OpA::PER;
            opa.template issue_part<(c0 < PA ? c0 : PA), (c1 < PA ? c1 : PA)>(
                A, p.lda, k0, As + dst * OpA::STAGE);
            opb.template issue_part<(c0 > PA ? c0 - PA : 0), (c1 > PA ? c1 - PA : 0)>(
                B, p.ldb, k0, Bs + dst * OpB::STAGE);
        };
        // Scheduling hint of group g with S = 3: the next group's reads, then
        // chunk g's copies.
        auto chunk_hint = [&](auto gc) __attribute__((always_inline)) {
            if (Cfg::ILV) {
                constexpr int kMfma = 4 * FM * FN;
                constexpr int kCopies = chunk_lo(decltype(gc)::value + 1) - chunk_lo(decltype(gc)::value);
                if constexpr (kCopies == 0) {
                    interleave_hint();
                } else {
                    front_hint<kMfma, kHintReads, kCopies, kMfma / 2>(
                        std::make_integer_sequence<int, kMfma>{});
                }
            }
        };
        // One K-tile of the steady state (tiles t+1 and t+2 exist and are
        // wholly inside K).  Nothing here branches, so each group's fragment
        // reads stay in one scheduling region with the MFMAs they are
        // interleaved with.
        auto ktile_steady = [&](int t, int cur) __attribute__((always_inline)) {
            const int nxt = next_stage(cur);
            const int dst = S == 2 ? cur : next_stage(nxt);  // tile t+2's stage
            const float* as = As + cur * OpA::STAGE;
            const float* bs = Bs + cur * OpB::STAGE;
            static_for<NGK - 1>([&](auto gc) __attribute__((always_inline)) {
                constexpr int g = decltype(gc)::value;
                __builtin_amdgcn_sched_barrier(0);
                read_group(as, bs, g0 + g + 1, (g + 1) & 1, t, No{});
                if constexpr (S == 3) copy_chunk(gc, (t + 2) * BK, dst);
                mfma_group(g & 1);
                if constexpr (S == 3) {
                    chunk_hint(gc);
                } else {
                    interleave_hint();
                }
                __builtin_amdgcn_sched_barrier(0);
            });
            // lgkmcnt(0), and tile t+1 landed (only tile t+2's copies issued
            // above may still be in flight)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(kPre) & ~(15 << 8));
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (S == 2) {
                // The copies of tile t+2 (into the stage every wave has
                // finished reading) and the first reads of tile t+1 are
                // spread between the last group's MFMAs.
                opa.issue_full(A, p.lda, (t + 2) * BK, As + dst * OpA::STAGE);
                opb.issue_full(B, p.ldb, (t + 2) * BK, Bs + dst * OpB::STAGE);
                read_group(As + nxt * OpA::STAGE, Bs + nxt * OpB::STAGE, g0, 0, t + 1, No{});
                mfma_group((NGK - 1) & 1);
                interleave_hint_copies();
            } else {
                read_group(As + nxt * OpA::STAGE, Bs + nxt * OpB::STAGE, g0, 0, t + 1, No{});
                copy_chunk(std::integral_constant<int, NGK - 1>{}, (t + 2) * BK, dst);
                mfma_group((NGK - 1) & 1);
                chunk_hint(std::integral_constant<int, NGK - 1>{});
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        // The last tiles (up to three), with run-time checks for the tile
        // that crosses K and for the end of K; tile t+2 is copied whole
        // after the barrier.
        auto read_rt = [&](const float* as, const float* bs, int g, int slot, int tile) {
            if (tile == tail_tile) {
                read_group(as, bs, g, slot, tile, Yes{});
            } else {
                read_group(as, bs, g, slot, tile, No{});
            }
        };
        auto ktile_last = [&](int t, int cur) {
            const int nxt = next_stage(cur);
            const int dst = S == 2 ? cur : next_stage(nxt);
            const float* as = As + cur * OpA::STAGE;
            const float* bs = Bs + cur * OpB::STAGE;
#pragma unroll
            for (int g = 0; g + 1 < NGK; ++g) {
                __builtin_amdgcn_sched_barrier(0);
                read_rt(as, bs, g0 + g + 1, (g + 1) & 1, t);
                mfma_group(g & 1);
                interleave_hint();
                __builtin_amdgcn_sched_barrier(0);
            }
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & ~(15 << 8));  // vmcnt(0) lgkmcnt(0)
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (t + 2 < ktiles) issue_tile(t + 2, dst);
            __builtin_amdgcn_sched_barrier(0);
            if (t + 1 < ktiles) {
                read_rt(As + nxt * OpA::STAGE, Bs + nxt * OpB::STAGE, g0, 0, t + 1);
            }
            mfma_group((NGK - 1) & 1);
            interleave_hint();
            __builtin_amdgcn_sched_barrier(0);
        };
        // Steady state while tile t+2 is not the last tile; a K that ends in
        // a full tile needs no checks until its last two tiles.
        const int steady = has_tail ? ktiles - 3 : ktiles - 2;
        int cur = 0;
        for (; t < steady; ++t) {
            ktile_steady(t, cur);
            cur = next_stage(cur);
        }
        for (; t < ktiles; ++t) {
            ktile_last(t, cur);
            cur = next_stage(cur);
        }
    } else if (NG % 2 == 0 && all_ahead && tail_tile < 0) {
        // Every tile is in its own stage, so the only wait before reading tile
        // t+1 is for its copies (each wave's own, then the barrier for the
        // others').  That wait and the first fragment reads of tile t+1 come
        // before the MFMAs of tile t's last group, so the reads' latency and
        // the barrier overlap those MFMAs instead of stalling the next tile.
        // Whole K-tiles only, and the tile count a template constant: with
        // straight-line code and no masking branch, each group's MFMAs wait
        // for that group's fragment reads alone (at a loop's back edge or a
        // branch the waits fall back to every outstanding read).
        auto run = [&](auto kt) __attribute__((always_inline)) {
            constexpr int KT = decltype(kt)::value;
            auto land = [&](auto tc) __attribute__((always_inline)) {
                constexpr int later = KT - 1 - decltype(tc)::value;  // in flight after it
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(later * PER_TILE));
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
            };
            auto read_tile_group = [&](int t, int g, int slot) __attribute__((always_inline)) {
                read_group(As + t * OpA::STAGE, Bs + t * OpB::STAGE, g, slot, t,
                           std::false_type{});
            };
            auto tile = [&](auto tc) __attribute__((always_inline)) {
                constexpr int t = decltype(tc)::value;
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    __builtin_amdgcn_sched_barrier(0);
                    // NG is even, so group 0 of tile t+1 takes slot (g + 1) & 1 = 0
                    if (g + 1 < NG) {
                        read_tile_group(t, g + 1, (g + 1) & 1);
                    } else if constexpr (t + 1 < KT) {
                        land(std::integral_constant<int, t + 1>{});
                        read_tile_group(t + 1, 0, 0);
                    }
                    if (!Cfg::ILV) __builtin_amdgcn_sched_barrier(0);
                    mfma_group(g & 1);
                    if (g + 1 < NG) interleave_hint();
                    __builtin_amdgcn_sched_barrier(0);
                }
            };
            land(std::integral_constant<int, 0>{});
            read_tile_group(0, 0, 0);
            tile(std::integral_constant<int, 0>{});
            if constexpr (KT > 1) tile(std::integral_constant<int, 1>{});
            if constexpr (KT > 2) tile(std::integral_constant<int, 2>{});
            if constexpr (KT > 3) tile(std::integral_constant<int, 3>{});
        };
        static_assert(S <= 4, "tile counts 1 to 4 below");
        if (ktiles == 1) {
            run(std::integral_constant<int, 1>{});
        } else if (ktiles == 2) {
            run(std::integral_constant<int, 2>{});
        } else if (S >= 3 && ktiles == 3) {
            run(std::integral_constant<int, (S >= 3 ? 3 : 1)>{});
        } else if (S >= 4) {
            run(std::integral_constant<int, (S >= 4 ? 4 : 1)>{});
        }
    } else {
        int stage = 0;
        for (int t = 0; t < ktiles; ++t) {
            // Loads of tiles t+1 .. t+S-2 may stay in flight; tile t's must land.
            const int later = min(S - 2, ktiles - 1 - t);
            if (S >= 4 && later >= 2) {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * PER_TILE));
            } else if (S >= 3 && later >= 1) {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(PER_TILE));
            } else {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            }
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (!all_ahead && t + S - 1 < ktiles) {
                issue_tile(t + S - 1, stage == 0 ? S - 1 : stage - 1);  // (t + S - 1) % S
            }
            const float* as = As + stage * OpA::STAGE;
            const float* bs = Bs + stage * OpB::STAGE;
            // This path (three or more stages) masks at run time.
            auto read_rt = [&](int g, int slot) {
                if (t == tail_tile) {
                    read_group(as, bs, g, slot, t, std::true_type{});
                } else {
                    read_group(as, bs, g, slot, t, std::false_type{});
                }
            };
            read_rt(0, 0);
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                __builtin_amdgcn_sched_barrier(0);
                if (g + 1 < NG) read_rt(g + 1, (g + 1) & 1);
                if (!Cfg::ILV) __builtin_amdgcn_sched_barrier(0);
                mfma_group(g & 1);
                if (g + 1 < NG) interleave_hint();
                __builtin_amdgcn_sched_barrier(0);
            }
            stage = stage + 1 == S ? 0 : stage + 1;
        }
    }

    if constexpr (KS > 1) {
        // The other sets' partial sums meet set 0's in LDS (the stages are
        // free: every copy has landed and every wave is past its last read),
        // added in set order.
        constexpr int kPart = FM * FN * 16 * kWave;  // floats of one wave's accumulators
        static_assert((KS - 1) * WMN * kPart <= S * (OpA::STAGE + OpB::STAGE),
                      "partial sums fit in the LDS stages");
        __syncthreads();
        if (kset > 0) {
            float* dst = lds + ((kset - 1) * WMN + wmn) * kPart + lane;
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
#pragma unroll
                    for (int r = 0; r < 16; ++r) dst[((mi * FN + ni) * 16 + r) * kWave] = acc[mi][ni][r];
        }
        __syncthreads();
        if (kset > 0) return;
#pragma unroll
        for (int ks = 1; ks < KS; ++ks) {
            const float* src = lds + ((ks - 1) * WMN + wmn) * kPart + lane;
#pragma unroll
            for (int mi = 0; mi < FM; ++mi)
#pragma unroll
                for (int ni = 0; ni < FN; ++ni)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        acc[mi][ni][r] += src[((mi * FN + ni) * 16 + r) * kWave];
        }
    }
    // Streaming (non-temporal) stores where C is large next to the work: the
    // 128- and 256-row tiles run only where C is at least about 8 MiB, and
    // the four-stage short-K tile (CfgDma64S, K <= 128) writes as many bytes
    // of C as it reads (the C4 batch: 5.57 -> 5.25 us in the trace; for the
    // 64x64 and 96x32 tiles of 777^3 to 2048^3 they measured -1% to +2%).
    constexpr int kStreamStores = ((BM >= 128 && BN >= 128) || S == 4) ? 1 : 0;
    store_wave_tile<FM, FN, kStreamStores>(acc, p, bz, m0 + wm0, n0 + wn0, half, l32, bias_pre);
}

// ---------------------------------------------------------------------------
// Small-problem kernel: one 32x32 tile of C per block, the K range split over
// KW waves.  Operands go straight from global (L2) into MFMA registers with
// the k index permuted inside each group of 8: at step s (0..3) the lane in
// half h supplies k = k0 + 4h + s, so one lane's four A values are contiguous
// (a 16-byte load when A is k-contiguous).  The permutation is applied to A
// and B alike, so the four MFMAs still cover k0..k0+7 exactly once.
// Groups are loaded ITS at a time into one of two register buffers: the loads
// of the next ITS groups are in flight while the MFMAs of the current ones
// run, so a wave pays the global-load latency about once per ITS groups
// instead of once per group.  Partial 32x32 sums meet in LDS and are added
// in wave order, then the epilogue runs.
// ---------------------------------------------------------------------------
// One group of 8 reduction steps for this lane.  `row` and `col` are already
// clamped into the matrix: a lane whose row (column) lies outside C loads a
// valid row and only pollutes accumulator rows (columns) that are never
// stored, so no select is needed and every load is issued unconditionally.
// With `tail`, k indices at or past kend are clamped and their values zeroed.
template <bool TA, bool TB, bool VA, bool VB>
__device__ __forceinline__ void splitk_load_group(const float* __restrict__ A,
                                                  const float* __restrict__ B,
                                                  const GemmParams& p, int row, int col,
                                                  int kb, int kend, bool tail, float a[4],
                                                  float b[4]) {
    if (!tail) {
        if (!TA) {
            const float* ar = A + (int64_t)row * p.lda + kb;
            if (VA) {
                const floatx4 v = *reinterpret_cast<const floatx4*>(ar);
                a[0] = v[0]; a[1] = v[1]; a[2] = v[2]; a[3] = v[3];
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) a[s] = ar[s];
            }
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) a[s] = A[(int64_t)(kb + s) * p.lda + row];
        }
        if (TB) {
            const float* br = B + (int64_t)col * p.ldb + kb;
            if (VB) {
                const floatx4 v = *reinterpret_cast<const floatx4*>(br);
                b[0] = v[0]; b[1] = v[1]; b[2] = v[2]; b[3] = v[3];
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) b[s] = br[s];
            }
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) b[s] = B[(int64_t)(kb + s) * p.ldb + col];
        }
    } else {
        float av[4], bv[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kk = kb + s < kend ? kb + s : 0;
            av[s] = TA ? A[(int64_t)kk * p.lda + row] : A[(int64_t)row * p.lda + kk];
            bv[s] = TB ? B[(int64_t)col * p.ldb + kk] : B[(int64_t)kk * p.ldb + col];
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bool kin = kb + s < kend;
            a[s] = kin ? av[s] : 0.0f;
            b[s] = kin ? bv[s] : 0.0f;
        }
    }
}

// The body takes its block index and the number of blocks that share the
// tile mapping explicitly, so a grouped launch can run it on a sub-range of
// its grid (sgemm_group_kernel).
// LATE_PRE issues the epilogue's operand loads after the first super-chunk's
// loads instead of before them: for a caller whose shape and operand
// addresses arrive in SGPRs, the epilogue's fields (C, its extra operand, the
// epilogue kind) are then the only scalar loads, and nothing waits for them
// before the first loads are issued.
template <int KW, int ITS, bool TA, bool TB, bool VA, bool VB, bool LATE_PRE = false>
__device__ __forceinline__ void splitk32_body(const GemmParams& p, int tiles_m, int tiles_n,
                                              int kchunk, int bid, int nblocks, int64_t bz) {
    __shared__ float red[KW][16][kWave];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    // Wave-uniform (scalar), so the K-range tests below are scalar branches:
    // computed as tid / 64 the compiler treats them as divergent, wraps the
    // loads in exec-masked branches and waits for every load of the wave's K
    // range before the first MFMA.
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int i = lane & 31;
    const int h = lane >> 5;

    int tm, tn;
    tile_coords(bid, nblocks, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * 32;
    const int n0 = tn * 32;
    const float* __restrict__ A = p.A + bz * p.strideA;
    const float* __restrict__ B = p.B + bz * p.strideB;

    // Row of op(A) and column of op(B) this lane feeds, clamped into the
    // matrix (see splitk_load_group).
    const int row = min(m0 + i, p.M - 1);
    const int col = min(n0 + i, p.N - 1);
    const int kbeg = wave * kchunk;
    const int kend = min(p.K, kbeg + kchunk);
    const int groups = kend > kbeg ? (kend - kbeg + 7) / 8 : 0;
    const int supers = (groups + ITS - 1) / ITS;

    float* __restrict__ C = p.C + bz * p.strideC;
    const float* __restrict__ aux = p.aux ? p.aux + bz * p.strideC : nullptr;
    float* __restrict__ upd = p.upd ? p.upd + bz * p.strideC : nullptr;
    // The epilogue's elements of this thread, and their extra operand,
    // fetched now (see epilogue_operand).
    constexpr int kEpi = (16 * kWave + KW * kWave - 1) / (KW * kWave);
    float pre[kEpi];
    auto load_pre = [&]() {
#pragma unroll
        for (int q = 0; q < kEpi; ++q) {
            const int e = tid + q * KW * kWave;
            const int r = e / kWave;
            const int ln = e % kWave;
            // Clamped into C rather than branched around: a lane-divergent
            // branch around the load makes both of its sides load into one
            // register, and the compiler then waits for the first before the
            // K loop's loads are even issued.  Out-of-range lanes load a
            // valid element they never store.
            const int gi = min(m0 + 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3), p.M - 1);
            const int gj = min(n0 + (ln & 31), p.N - 1);
            pre[q] = epilogue_operand(p, C, aux, upd, (int64_t)gi * p.ldc + gj, gj);
        }
    };
    if constexpr (!LATE_PRE) load_pre();

    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

    float a0[ITS][4], b0[ITS][4], a1[ITS][4], b1[ITS][4];
    // Groups past the wave's range load as zeros, so a super-chunk always
    // issues ITS groups of MFMAs.
    auto load_super = [&](int sc, float (&a)[ITS][4], float (&b)[ITS][4]) {
        const int k0 = kbeg + 8 * sc * ITS;
        if (k0 + 8 * ITS <= kend) {  // wave-uniform: the whole super-chunk is in range
#pragma unroll
            for (int q = 0; q < ITS; ++q)
                splitk_load_group<TA, TB, VA, VB>(A, B, p, row, col, k0 + 8 * q + 4 * h, kend,
                                                  false, a[q], b[q]);
        } else {
#pragma unroll
            for (int q = 0; q < ITS; ++q)
                splitk_load_group<TA, TB, VA, VB>(A, B, p, row, col, k0 + 8 * q + 4 * h, kend,
                                                  true, a[q], b[q]);
        }
    };
    auto mfma_super = [&](const float (&a)[ITS][4], const float (&b)[ITS][4]) {
#pragma unroll
        for (int q = 0; q < ITS; ++q)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q][s], b[q][s], acc, 0, 0, 0);
    };

    if (supers > 0) load_super(0, a0, b0);
    if constexpr (LATE_PRE) load_pre();
    for (int sc = 0; sc < supers; sc += 2) {
        if (sc + 1 < supers) load_super(sc + 1, a1, b1);
        mfma_super(a0, b0);
        if (sc + 1 < supers) {
            if (sc + 2 < supers) load_super(sc + 2, a0, b0);
            mfma_super(a1, b1);
        }
    }

#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();

    float v[kEpi];
    int64_t off[kEpi];
    bool live[kEpi];
#pragma unroll
    for (int q = 0; q < kEpi; ++q) {
        const int e = tid + q * KW * kWave;
        const int r = (e / kWave) & 15;
        const int ln = e % kWave;
        v[q] = 0.0f;
#pragma unroll
        for (int w = 0; w < KW; ++w) v[q] += red[w][r][ln];
        const int gi = m0 + 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3);
        const int gj = n0 + (ln & 31);
        live[q] = e < 16 * kWave && gi < p.M && gj < p.N;
        off[q] = (int64_t)gi * p.ldc + gj;
    }
    store_epilogue_elems<kEpi>(v, off, live, pre, p, C, upd);
}

// The operands' addresses, leading dimensions, 32-bit batch strides, shape and
// K chunk come as leading scalar arguments, preloaded in SGPRs (14 dwords;
// the compiler preloads only leading arguments that are not aggregates), so
// the first loads wait for no scalar load of the GemmParams aggregate, which
// supplies the epilogue's fields; its operand is loaded after the first loads
// (LATE_PRE).  The tile counts and the grid's size follow from the shape.
template <int KW, int ITS, bool TA, bool TB, bool VA, bool VB>
__global__ void __launch_bounds__(KW * 64)
sgemm_splitk32_kernel(const float* __restrict__ A0, const float* __restrict__ B0, int64_t lda,
                      int64_t ldb, int strideA, int strideB, int M, int N, int K, int kchunk,
                      GemmParams pa) {
    GemmParams p = pa;
    p.A = A0;
    p.B = B0;
    p.lda = lda;
    p.ldb = ldb;
    p.strideA = strideA;
    p.strideB = strideB;
    p.M = M;
    p.N = N;
    p.K = K;
    const int tiles_m = (M + 31) / 32, tiles_n = (N + 31) / 32;
    splitk32_body<KW, ITS, TA, TB, VA, VB, true>(p, tiles_m, tiles_n, kchunk, blockIdx.x,
                                                 tiles_m * tiles_n, blockIdx.y);
}

// ---------------------------------------------------------------------------
// Small-problem kernel with 16x16 output tiles (v_mfma_f32_16x16x4_f32), for
// outputs too small to give 32x32 tiles to every CU.  Lane layout:
//   operand a: lane l supplies A[i = l % 16][kk = l / 16]
//   operand b: lane l supplies B[kk = l / 16][j = l % 16]
//   result   : lane l, register r holds D[4 * (l / 16) + r][l % 16]
// A group covers 16 reduction steps: at step s (0..3) the lane in quarter q
// supplies k = k0 + 4q + s (the same permutation for A and B), so a lane's
// four A values are contiguous.  K is split over KW waves; groups are loaded
// ITS at a time into two alternating register buffers; partials meet in LDS.
// ---------------------------------------------------------------------------
template <bool TA, bool TB, bool VA, bool VB>
__device__ __forceinline__ void splitk16_load_group(const float* __restrict__ A,
                                                    const float* __restrict__ B,
                                                    const GemmParams& p, int row, int col,
                                                    int kb, int kend, bool tail, float a[4],
                                                    float b[4]) {
    // Same contract as splitk_load_group: row/col are clamped into the matrix.
    splitk_load_group<TA, TB, VA, VB>(A, B, p, row, col, kb, kend, tail, a, b);
}

// The body takes its block index and the number of blocks that share the
// tile mapping explicitly, so a grouped launch can run it on a sub-range of
// its grid (sgemm_group_kernel), as splitk32_body does.
template <int KW, int ITS, bool TA, bool TB, bool VA, bool VB>
__device__ __forceinline__ void splitk16_body(const GemmParams& p, int tiles_m, int tiles_n,
                                              int kchunk, int bid, int nblocks, int64_t bz) {
    __shared__ float red[KW][4][kWave];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    // wave-uniform, so the K-range tests are scalar branches (see splitk32_body)
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int i = lane & 15;
    const int q = lane >> 4;

    int tm, tn;
    tile_coords(bid, nblocks, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * 16;
    const int n0 = tn * 16;
    const float* __restrict__ A = p.A + bz * p.strideA;
    const float* __restrict__ B = p.B + bz * p.strideB;

    float* __restrict__ C = p.C + bz * p.strideC;
    const float* __restrict__ aux = p.aux ? p.aux + bz * p.strideC : nullptr;
    float* __restrict__ upd = p.upd ? p.upd + bz * p.strideC : nullptr;
    // The epilogue's elements of this thread and their extra operand, fetched
    // now (see epilogue_operand).
    constexpr int kEpi = (4 * kWave + KW * kWave - 1) / (KW * kWave);
    float pre[kEpi];
#pragma unroll
    for (int u = 0; u < kEpi; ++u) {
        const int e = tid + u * KW * kWave;
        const int r = e / kWave;
        const int ln = e % kWave;
        // Clamped, not branched around (see splitk32_body).
        const int gi = min(m0 + 4 * (ln >> 4) + r, p.M - 1);
        const int gj = min(n0 + (ln & 15), p.N - 1);
        pre[u] = epilogue_operand(p, C, aux, upd, (int64_t)gi * p.ldc + gj, gj);
    }

    const int row = min(m0 + i, p.M - 1);
    const int col = min(n0 + i, p.N - 1);
    const int kbeg = wave * kchunk;
    const int kend = min(p.K, kbeg + kchunk);
    const int groups = kend > kbeg ? (kend - kbeg + 15) / 16 : 0;
    const int supers = (groups + ITS - 1) / ITS;

    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float a0[ITS][4], b0[ITS][4], a1[ITS][4], b1[ITS][4];
    auto load_super = [&](int sc, float (&a)[ITS][4], float (&b)[ITS][4]) {
        const int k0 = kbeg + 16 * sc * ITS;
        if (k0 + 16 * ITS <= kend) {
#pragma unroll
            for (int g = 0; g < ITS; ++g)
                splitk16_load_group<TA, TB, VA, VB>(A, B, p, row, col, k0 + 16 * g + 4 * q, kend,
                                                    false, a[g], b[g]);
        } else {
#pragma unroll
            for (int g = 0; g < ITS; ++g)
                splitk16_load_group<TA, TB, VA, VB>(A, B, p, row, col, k0 + 16 * g + 4 * q, kend,
                                                    true, a[g], b[g]);
        }
    };
    auto mfma_super = [&](const float (&a)[ITS][4], const float (&b)[ITS][4]) {
#pragma unroll
        for (int g = 0; g < ITS; ++g)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[g][s], b[g][s], acc, 0, 0, 0);
    };

    if (supers > 0) load_super(0, a0, b0);
    for (int sc = 0; sc < supers; sc += 2) {
        if (sc + 1 < supers) load_super(sc + 1, a1, b1);
        mfma_super(a0, b0);
        if (sc + 1 < supers) {
            if (sc + 2 < supers) load_super(sc + 2, a0, b0);
            mfma_super(a1, b1);
        }
    }

#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();

#pragma unroll
    for (int u = 0; u < kEpi; ++u) {
        const int e = tid + u * KW * kWave;
        if (e >= 4 * kWave) break;
        const int r = e / kWave;
        const int ln = e % kWave;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < KW; ++w) v += red[w][r][ln];
        const int gi = m0 + 4 * (ln >> 4) + r;
        const int gj = n0 + (ln & 15);
        if (gi < p.M && gj < p.N) {
            store_epilogue_pre(v, p, C, upd, (int64_t)gi * p.ldc + gj, pre[u]);
        }
    }
}

template <int KW, int ITS, bool TA, bool TB, bool VA, bool VB>
__global__ void __launch_bounds__(KW * 64)
sgemm_splitk16_kernel(const float* __restrict__ A0, const float* __restrict__ B0, int64_t lda,
                      int64_t ldb, int strideA, int strideB, int M, int N, int K, int kchunk,
                      GemmParams pa) {
    // (leading scalar arguments as sgemm_splitk32_kernel's; the epilogue's
    // operand is loaded before the K range here: after the first loads it
    // measured slower, 3.93 -> 4.09 us at 256x256x512 with bias+ReLU)
    GemmParams p = pa;
    p.A = A0;
    p.B = B0;
    p.lda = lda;
    p.ldb = ldb;
    p.strideA = strideA;
    p.strideB = strideB;
    p.M = M;
    p.N = N;
    p.K = K;
    const int tiles_m = (M + 15) / 16, tiles_n = (N + 15) / 16;
    splitk16_body<KW, ITS, TA, TB, VA, VB>(p, tiles_m, tiles_n, kchunk, blockIdx.x,
                                           tiles_m * tiles_n, blockIdx.y);
}

// ---------------------------------------------------------------------------
// sgemm_splitk16_kernel with its operands staged in LDS by direct-to-LDS
// copies, for the NN layout with 16-byte-aligned rows of A and B (N % 4 == 0)
// and a K range of KC = 64 per wave (768 < K <= 1024 at KW = 16).  Wave w
// copies the 16 x KC panel of A and the KC x 16 panel of B of its own K range
// into its own LDS region, every copy issued at once (no registers hold the
// bytes in flight), and waits only for its own copies, a 16-k group at a
// time (the MFMAs of a group run while later groups land).  Its MFMAs run
// the register kernel's sequence (same K ranges, k order and wave order of
// the final sums), so the results are that kernel's bit for bit.
// LDS images, per wave:
//  * A: group-major, GR groups of 16 rows x 16 k (one 1 KB copy each); in a
//    group the 16-byte chunk c of row r sits in slot c ^ kc_swz16(r), so a
//    ds_read_b128 of 16 rows x one chunk spreads over the banks.
//  * B: KC rows of 16 floats, in groups of 16 k; within a group slot row
//    4s + q holds k = 4q + s, so the ds_read_b32 of MFMA step s (lane quarter
//    q reads k = 4q + s) covers 64 consecutive floats.
// Rows past M, columns past N and k past K copy clamped, in-bounds elements;
// k past K is zeroed before its MFMA, the rest reach only unstored outputs.
// The block has one wave per KC of K (at most KW); the register form's idle
// waves only added +0.0 to each sum, so the results are still its bits.
// ---------------------------------------------------------------------------
template <int KW, int KC>
__global__ void __launch_bounds__(KW * 64)
sgemm_splitk16_lds_kernel(const float* __restrict__ A0, const float* __restrict__ B0,
                          int64_t strideA, int64_t strideB, int lda, int ldb, int M, int N, int K,
                          GemmParams p) {
    constexpr int GR = KC / 16;           // k groups of a wave
    static_assert(KC == 64 && GR == 4, "copy counts and waits assume KC = 64 (four groups)");
    // One array per k group (A's 16 x 16 floats, then B's 16 x 16), so that
    // the compiler sees a group's reads alias only that group's copies and
    // waits for those alone (with one array it waits for every copy).
    __shared__ __attribute__((aligned(16))) float lg0[KW][512];
    __shared__ __attribute__((aligned(16))) float lg1[KW][512];
    __shared__ __attribute__((aligned(16))) float lg2[KW][512];
    __shared__ __attribute__((aligned(16))) float lg3[KW][512];
    __shared__ float red[KW][4][kWave];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int i = lane & 15;
    const int q = lane >> 4;

    int tm, tn;
    // (the grid is exactly the tiles: their count stands in for gridDim.x,
    // which would be a scalar load from the dispatch's implicit arguments)
    const int tiles_m = (M + 15) / 16, tiles_n = (N + 15) / 16;
    tile_coords(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * 16;
    const int n0 = tn * 16;
    const int64_t bz = blockIdx.y;
    // The operands' shape and addresses come as leading scalar arguments,
    // which the kernel receives preloaded in SGPRs; fields of the GemmParams
    // aggregate are not preloaded, and the copies would wait for a scalar
    // load of them.  `p` supplies the rest (C, the epilogue).
    const float* __restrict__ A = A0 + bz * strideA;
    const float* __restrict__ B = B0 + bz * strideB;

    // The block has exactly one wave per KC of K (the launch sizes it so), so
    // every wave's K range starts inside K.  (The count comes from K rather
    // than blockDim.x, another scalar load from the implicit arguments.)
    const int nw = (K + KC - 1) / KC;
    const int kbeg = wave * KC;
    auto region = [&](auto gc) -> float* {
        constexpr int g = decltype(gc)::value;
        if constexpr (g == 0) return lg0[wave];
        else if constexpr (g == 1) return lg1[wave];
        else if constexpr (g == 2) return lg2[wave];
        else return lg3[wave];
    };
    // The epilogue's element of this thread (the first four waves) and its
    // extra operand (see epilogue_operand), loaded after the copies: its
    // address needs the aggregate's fields, and the copies need only the
    // preloaded arguments.
    constexpr int kEpi = 1;
    float pre[kEpi];
    float* __restrict__ C = nullptr;
    const float* __restrict__ aux = nullptr;
    float* __restrict__ upd = nullptr;
    auto load_pre = [&]() {
        // (the barrier keeps the wait for the aggregate's fields after the
        // copies: scheduled earlier, it would hold them back)
        __builtin_amdgcn_sched_barrier(0);
        C = p.C + bz * p.strideC;
        aux = p.aux ? p.aux + bz * p.strideC : nullptr;
        upd = p.upd ? p.upd + bz * p.strideC : nullptr;
#pragma unroll
        for (int u = 0; u < kEpi; ++u) {
            const int e = tid;
            const int r = e / kWave;
            const int ln = e % kWave;
            const int gi = min(m0 + 4 * (ln >> 4) + r, M - 1);
            const int gj = min(n0 + (ln & 15), N - 1);
            pre[u] = epilogue_operand(p, C, aux, upd, (int64_t)gi * p.ldc + gj, gj);
        }
    };
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    {
        // Copies in group order, A's then B's of each group, so group g has
        // landed once at most 2 (GR - 1 - g) copies are outstanding.
        const int ar = lane >> 2;             // A: row of this lane's chunk
        const int aq = lane & 3;              // A: slot within the row's group
        const int ac = aq ^ kc_swz16(ar);     // A: the chunk (k / 4 in the group) it holds
        const int arow = min(m0 + ar, M - 1) - m0;
        const int sr = lane >> 2;             // B: slot row of the group
        const int kr = 4 * (sr & 3) + (sr >> 2);
        const int bcol = min(n0 + 4 * (lane & 3), N - 4) - n0;
        // Buffer copies from wave-uniform bases (the block's first row of A,
        // the wave's first k row of B); the lane parts are 32-bit offsets
        // (the host keeps 16 rows of A and 64 rows of B below 2 GiB).
        const __amdgpu_buffer_rsrc_t ra = dma_buffer(wave_uniform(A + (int64_t)m0 * lda));
        const __amdgpu_buffer_rsrc_t rb =
            dma_buffer(wave_uniform(B + (int64_t)kbeg * ldb + n0));
        auto copy = [&](auto gc) {
            constexpr int g = decltype(gc)::value;
            const int gk = min(kbeg + 16 * g + 4 * ac, K - 4);
            dma_buf_copy16(ra, (uint32_t)((int64_t)arow * lda + gk) * 4u, region(gc));
            const int bk = min(kbeg + 16 * g + kr, K - 1) - kbeg;
            dma_buf_copy16(rb, (uint32_t)((int64_t)bk * ldb + bcol) * 4u,
                           region(gc) + 4 * kWave);
        };
        copy(std::integral_constant<int, 0>{});
        copy(std::integral_constant<int, 1>{});
        copy(std::integral_constant<int, 2>{});
        copy(std::integral_constant<int, 3>{});
        load_pre();
        // Nothing may move between the copies and the waits below.
        __builtin_amdgcn_sched_barrier(0);
        // Group g's MFMAs start as soon as its two copies have landed.  Loads
        // complete in order and the epilogue operand was loaded after the
        // copies, so once at most 2 (GR - 1 - g) + 1 operations (the later
        // groups' copies and that load) are outstanding, group g's have
        // landed; the wait is written here rather than left to the compiler,
        // which places the same one only because it tells the four arrays
        // apart.
        auto group = [&](auto gc) {
            constexpr int g = decltype(gc)::value;
            // (the barrier keeps the scheduler from lifting this wait above
            // the previous group's MFMAs)
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * (GR - 1 - g) + 1));
            const int k0 = kbeg + 16 * g;
            if (k0 >= K) return;
            const float* as = region(gc);
            const float* bs = as + 4 * kWave;
            floatx4 a = *reinterpret_cast<const floatx4*>(as + i * 16 + 4 * (q ^ kc_swz16(i)));
            float b[4];
#pragma unroll
            for (int st = 0; st < 4; ++st) b[st] = bs[(4 * st + q) * 16 + i];
            if (k0 + 16 > K) {
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    const bool in = k0 + 4 * q + st < K;
                    a[st] = in ? a[st] : 0.0f;
                    b[st] = in ? b[st] : 0.0f;
                }
            }
#pragma unroll
            for (int st = 0; st < 4; ++st)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st], b[st], acc, 0, 0, 0);
        };
        group(std::integral_constant<int, 0>{});
        group(std::integral_constant<int, 1>{});
        group(std::integral_constant<int, 2>{});
        group(std::integral_constant<int, 3>{});
    }

#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();

#pragma unroll
    for (int u = 0; u < kEpi; ++u) {
        const int e = tid;
        if (e >= 4 * kWave) break;
        const int r = e / kWave;
        const int ln = e % kWave;
        float v = 0.0f;
        for (int w = 0; w < nw; ++w) v += red[w][r][ln];
        const int gi = m0 + 4 * (ln >> 4) + r;
        const int gj = n0 + (ln & 15);
        if (gi < M && gj < N) {
            store_epilogue_pre(v, p, C, upd, (int64_t)gi * p.ldc + gj, pre[u]);
        }
    }
}

// ---------------------------------------------------------------------------
// Skinny kernel for M <= MR (MR <= 8) with B not transposed: a bandwidth
// kernel whose cost is one pass over B.  A block of NT threads owns a strip of
// STRIP columns and the whole K range: CL lanes across the strip (float4 each
// when VB) and KL = NT / CL lanes along K.  Each lane issues UNR rows of B
// before using any (UNR independent 16-byte loads in flight per lane), keeps
// MR x CW partial sums in registers, and the KL partials meet in LDS, added in
// lane order.  Strips are renumbered so the 8 XCDs each stream one contiguous
// band of B's columns.  Column and row indices are clamped into the matrices:
// lanes past the edge load valid data that only reaches outputs never stored.
// ---------------------------------------------------------------------------
// The operands' addresses, leading dimensions, 32-bit batch strides, shape and
// strip count lead the arguments, preloaded in SGPRs (see
// sgemm_splitk32_kernel); the aggregate supplies the epilogue.
template <int MR, bool TA, bool VB, int STRIP, int NT, int UNR>
__global__ void __launch_bounds__(NT)
sgemm_skinny_kernel(const float* __restrict__ A0, const float* __restrict__ B0, int64_t lda,
                    int64_t ldb, int strideA, int strideB, int M, int N, int K, int strips,
                    GemmParams pa) {
    GemmParams p = pa;
    p.A = A0;
    p.B = B0;
    p.lda = lda;
    p.ldb = ldb;
    p.strideA = strideA;
    p.strideB = strideB;
    p.M = M;
    p.N = N;
    p.K = K;
    constexpr int CW = VB ? 4 : 1;
    constexpr int CL = STRIP / CW;
    constexpr int KL = NT / CL;
    __shared__ float red[KL][MR][STRIP];

    const int tid = threadIdx.x;
    const int cl = tid % CL;
    const int kl = tid / CL;

    int sid = blockIdx.x;
    if ((strips & 7) == 0) sid = (sid & 7) * (strips >> 3) + (sid >> 3);
    const int64_t bz = blockIdx.y;
    const float* __restrict__ A = p.A + bz * p.strideA;
    const float* __restrict__ B = p.B + bz * p.strideB;
    // VB: N % 4 == 0, so clamping to the last float4 keeps whole vectors.
    const int n0 = min(sid * STRIP + cl * CW, p.N - CW);

    float acc[MR][CW];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < CW; ++c) acc[m][c] = 0.0f;

    auto a_at = [&](int m, int k) {
        const int mm = min(m, M - 1);
        return TA ? A[(int64_t)k * p.lda + mm] : A[(int64_t)mm * p.lda + k];
    };
    auto b_at = [&](int k, float (&b)[CW]) {
        if (VB) {
            const floatx4 v = *reinterpret_cast<const floatx4*>(B + (int64_t)k * p.ldb + n0);
#pragma unroll
            for (int c = 0; c < CW; ++c) b[c] = v[c];
        } else {
            b[0] = B[(int64_t)k * p.ldb + n0];
        }
    };

    int k = kl;
    for (; k + (UNR - 1) * KL < K; k += UNR * KL) {
        float b[UNR][CW];
        float a[UNR][MR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) b_at(k + u * KL, b[u]);
#pragma unroll
        for (int u = 0; u < UNR; ++u)
#pragma unroll
            for (int m = 0; m < MR; ++m) a[u][m] = a_at(m, k + u * KL);
#pragma unroll
        for (int u = 0; u < UNR; ++u)
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int c = 0; c < CW; ++c) acc[m][c] = fmaf(a[u][m], b[u][c], acc[m][c]);
    }
    for (; k < K; k += KL) {
        float b[CW];
        b_at(k, b);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float a = a_at(m, k);
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
    float* __restrict__ upd = p.upd ? p.upd + bz * p.strideC : nullptr;
    for (int e = tid; e < MR * STRIP; e += NT) {
        const int m = e / STRIP;
        const int c = e % STRIP;
        const int j = sid * STRIP + c;
        if (m < M && j < p.N) {
            float v = 0.0f;
            for (int q = 0; q < KL; ++q) v += red[q][m][c];
            const int64_t off = (int64_t)m * p.ldc + j;
            store_epilogue(v, p, C, aux, upd, off, j);
        }
    }
}

// ---------------------------------------------------------------------------
// K-split form of the skinny kernel, run when the caller supplies a workspace
// (one problem, B not transposed, 16-byte-vectorisable B).  When B's row
// pitch is a power of two (N = 4096: 16 KB) the strip kernel's blocks, each
// held to one 64-byte column piece of every row, stream at uneven rates: the
// pieces at some offsets within each 1 KB of a row are served much more
// slowly than the rest, so a few blocks finish long after the median.  Here a
// block owns a band of 256 columns (1 KB of each row, every offset) and a
// slice of K, so every block sees the same mix of offsets.  The price is a
// second, small pass.
//
// Pass 1 (skinny_part): block (band, slice) streams rows [k0, k1) of its band
// with four waves, each wave reading whole 1 KB row pieces (a lane a float4)
// with UNR rows in flight, the wave's rows interleaved by 4.  The four waves'
// sums meet in LDS, added in wave order, and the block writes its MR x 256
// partial to part[band][slice] in the workspace.
// Pass 2 (skinny_sum): one thread per output element adds its band's slices
// in slice order and applies the epilogue.  Both orders are fixed, so results
// repeat bit for bit.
// ---------------------------------------------------------------------------
constexpr int kSplitWaves = 4;
constexpr int kPartMaxRows = 512;  // slice rows whose A values the partial pass stages in LDS
constexpr int64_t kSplitMinElems = int64_t(1) << 23;   // 32 MB of B

// The pass takes only scalar arguments, which arrive preloaded in SGPRs (a
// GemmParams aggregate's fields would be scalar loads that the first loads
// wait for); `tiles` is the grid's size (bands x S).
template <int MR, bool TA, int UNR>
__global__ void __launch_bounds__(kSplitWaves * kWave)
sgemm_skinny_part_kernel(const float* __restrict__ A, const float* __restrict__ B,
                         float* __restrict__ part, int lda, int ldb, int M, int N, int K, int S,
                         int rows, int tiles) {
    constexpr int NW = kSplitWaves;
    __shared__ float red[NW][MR][kSplitBand];
    // A's slice for MR > 2 (see below); MR <= 2 keeps A in scalar loads
    __shared__ __attribute__((aligned(16))) float as_lds[MR > 2 ? kPartMaxRows * MR : 1];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    // wave-uniform, so A's loads below have wave-uniform addresses
    const int w = __builtin_amdgcn_readfirstlane(tid / kWave);

    int t = blockIdx.x;
    // each XCD takes a contiguous range of (band, slice) tiles: whole bands
    if ((tiles & 7) == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);
    const int band = t / S;
    const int slice = t - band * S;
    const int k0 = slice * rows;
    const int k1 = min(k0 + rows, K);
    // N % 4 == 0 here; lanes past the edge re-read the last float4 and their
    // sums land only in partial slots that pass 2 never reads.
    const int n0 = min(band * kSplitBand + lane * 4, N - 4);

    float acc[MR][4];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[m][c] = 0.0f;
    auto a_at = [&](int m, int k) {
        const int mm = min(m, M - 1);
        return TA ? A[(int64_t)k * (int64_t)lda + mm] : A[(int64_t)mm * (int64_t)lda + k];
    };

    auto load = [&](int kk, floatx4 (&b)[UNR], float (&a)[UNR][MR]) {
#pragma unroll
        for (int u = 0; u < UNR; ++u)
            b[u] = *reinterpret_cast<const floatx4*>(B + (int64_t)(kk + NW * u) * (int64_t)ldb + n0);
#pragma unroll
        for (int u = 0; u < UNR; ++u)
#pragma unroll
            for (int m = 0; m < MR; ++m) a[u][m] = a_at(m, kk + NW * u);
    };
    auto fma_rows = [&](const floatx4 (&b)[UNR], const float (&a)[UNR][MR]) {
#pragma unroll
        for (int u = 0; u < UNR; ++u)
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[m][c] = fmaf(a[u][m], b[u][c], acc[m][c]);
    };
    int k = k0 + w;
    if constexpr (MR <= 2) {
        // Software-pipelined: the next UNR rows are in flight while this
        // group's FMAs run (C5a M = 1: 15.9 -> 15.7 us; M = 1, N = 1024,
        // K = 16384: 18.9 -> 17.6 us).  At M = 8 the second register set
        // cost more than it hid (18.9 -> 23.5 us), so larger M keep one.
        const int span = k1 - k - NW * (UNR - 1);
        const int groups = span > 0 ? (span + NW * UNR - 1) / (NW * UNR) : 0;
        floatx4 b0[UNR], b1[UNR];
        float a0[UNR][MR], a1[UNR][MR];
        if (groups > 0) load(k, b0, a0);
        int it = 0;
        for (; it + 2 <= groups; it += 2) {
            load(k + NW * UNR, b1, a1);
            fma_rows(b0, a0);
            k += NW * UNR;
            if (it + 2 < groups) load(k + NW * UNR, b0, a0);
            fma_rows(b1, a1);
            k += NW * UNR;
        }
        if (it < groups) {
            fma_rows(b0, a0);
            k += NW * UNR;
        }
    } else if (rows <= kPartMaxRows) {
        // Larger M: A's slice (rows x MR floats) is staged in LDS once, so
        // the loop's only global loads are B's and its rows are software-
        // pipelined as above (with A in scalar loads the loop waited for all
        // of a group's MR * UNR A values, one cache round trip per group, and
        // a second set of them did not fit).  Same k order and sums, so the
        // same bits.  B's first rows are requested before the staging, so
        // their round trip overlaps A's instead of following the barrier.
        auto load_b = [&](int kk, floatx4 (&b)[UNR]) {
#pragma unroll
            for (int u = 0; u < UNR; ++u)
                b[u] = *reinterpret_cast<const floatx4*>(B + (int64_t)(kk + NW * u) * (int64_t)ldb + n0);
        };
        const int span = k1 - k - NW * (UNR - 1);
        const int groups = span > 0 ? (span + NW * UNR - 1) / (NW * UNR) : 0;
        floatx4 b0[UNR], b1[UNR];
        if (groups > 0) load_b(k, b0);
        // A's slice, all of a thread's loads issued before its first store
        // (one round trip).  Thread tid takes elements e = tid + 256 i of the
        // LDS image (k row e / MR, column e % MR), so a wave's stores are 64
        // consecutive floats, free of bank conflicts (with lanes along k they
        // were MR floats apart: 8-way conflicts at MR = 8).
        const int nrows = k1 - k0;
        constexpr int kThreads = NW * kWave;
        constexpr int kStagePer = kPartMaxRows * MR / kThreads;
        static_assert(kPartMaxRows * MR % kThreads == 0, "staging in whole passes");
        auto stage_pos = [&](int i, int& kk, int& m) {
            const int e = tid + i * kThreads;
            kk = e / MR;
            m = e % MR;
        };
        float av[kStagePer];
#pragma unroll
        for (int i = 0; i < kStagePer; ++i) {
            int kk, m;
            stage_pos(i, kk, m);
            av[i] = kk < nrows ? a_at(m, k0 + kk) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kStagePer; ++i) {
            int kk, m;
            stage_pos(i, kk, m);
            if (kk < nrows) as_lds[kk * MR + m] = av[i];
        }
        __syncthreads();
        auto fma_lds = [&](int kk, const floatx4 (&b)[UNR]) {
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
                const float* ar = as_lds + (kk + NW * u - k0) * MR;
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[m][c] = fmaf(ar[m], b[u][c], acc[m][c]);
            }
        };
        int it = 0;
        for (; it + 2 <= groups; it += 2) {
            load_b(k + NW * UNR, b1);
            fma_lds(k, b0);
            k += NW * UNR;
            if (it + 2 < groups) load_b(k + NW * UNR, b0);
            fma_lds(k, b1);
            k += NW * UNR;
        }
        if (it < groups) {
            fma_lds(k, b0);
            k += NW * UNR;
        }
    } else {
        for (; k + NW * (UNR - 1) < k1; k += NW * UNR) {
            floatx4 b[UNR];
            float a[UNR][MR];
            load(k, b, a);
            fma_rows(b, a);
        }
    }
    for (; k < k1; k += NW) {
        const floatx4 b = *reinterpret_cast<const floatx4*>(B + (int64_t)k * (int64_t)ldb + n0);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float a = a_at(m, k);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[m][c] = fmaf(a, b[c], acc[m][c]);
        }
    }

#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < 4; ++c) red[w][m][lane * 4 + c] = acc[m][c];
    __syncthreads();
    float* __restrict__ mine = part + (int64_t)t * MR * kSplitBand;
    for (int e = tid; e < MR * kSplitBand; e += NW * kWave) {
        const int m = e / kSplitBand;
        const int c = e % kSplitBand;
        float v = red[0][m][c];
#pragma unroll
        for (int q = 1; q < NW; ++q) v += red[q][m][c];
        mine[e] = v;
    }
}

// All SMAX loads are issued before the first add (slices past S re-read the
// last one and are not added), so the pass costs one memory round trip.
template <int MR, int SMAX>
__global__ void __launch_bounds__(kSplitBand)
sgemm_skinny_sum_kernel(const float* __restrict__ part, int S, int N, GemmParams p) {
    // (the partials' address, S and N lead the arguments, preloaded in SGPRs:
    // the loads below wait for no scalar load of the aggregate)
    const int band = blockIdx.x;
    const int m = blockIdx.y;
    const int j = band * kSplitBand + (int)threadIdx.x;
    if (j >= N) return;
    const float* __restrict__ src = part + ((int64_t)band * S * MR + m) * kSplitBand + threadIdx.x;
    float x[SMAX];
#pragma unroll
    for (int u = 0; u < SMAX; ++u) x[u] = src[(int64_t)min(u, S - 1) * MR * kSplitBand];
    float v = 0.0f;
#pragma unroll
    for (int u = 0; u < SMAX; ++u) v += u < S ? x[u] : 0.0f;
    store_epilogue(v, p, p.C, p.aux, p.upd, (int64_t)m * p.ldc + j, j);
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

// Batched problems of at most this many tiles each run on a 1-D grid whose
// blocks are spread so that each XCD owns whole batches (flat_batch_coords);
// larger ones keep grid.y = batch and the per-problem tile grouping.
constexpr int kFlatBatchMaxTiles = 64;

// Kernels that take the batch strides as 32-bit arguments run a batch whose
// stride does not fit one problem per launch: launch(q) for each.
inline bool strides_fit32(const GemmParams& p, int nbatch) {
    return nbatch <= 1 || (p.strideA <= INT32_MAX && p.strideB <= INT32_MAX);
}
template <class F>
hipError_t launch_per_problem(const GemmParams& p, int nbatch, F launch) {
    for (int b = 0; b < nbatch; ++b) {
        GemmParams q = p;
        q.A += b * p.strideA;
        q.B += b * p.strideB;
        q.C += b * p.strideC;
        if (q.aux) q.aux += b * p.strideC;
        if (q.upd) q.upd += b * p.strideC;
        const hipError_t err = launch(q);
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

template <class Cfg>
hipError_t launch_dma(const GemmParams& p, bool ta, bool tb, int nbatch, hipStream_t stream) {
    if (!strides_fit32(p, nbatch)) {
        return launch_per_problem(p, nbatch, [&](const GemmParams& q) {
            return launch_dma<Cfg>(q, ta, tb, 1, stream);
        });
    }
    const int tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;
    const int tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    const int tiles = tiles_m * tiles_n;
    const bool flat = nbatch > 1 && tiles <= kFlatBatchMaxTiles;
    const dim3 grid = flat ? dim3(tiles * nbatch) : dim3(tiles, nbatch);
    const dim3 block(Cfg::NT);
    const int sa = nbatch > 1 ? (int)p.strideA : 0;
    const int sb = nbatch > 1 ? (int)p.strideB : 0;
    const int mode = p.epilogue | (flat ? nbatch << 8 : 0);
#define FDL_DMA_LAUNCH(TA_, TB_)                                                              \
    hipLaunchKernelGGL((sgemm_dma_kernel<Cfg, TA_, TB_>), grid, block, 0, stream, p.A, p.B,   \
                       p.bias, sa, sb, (int)p.lda, (int)p.ldb, p.M, p.N, p.K, mode, p)
    if (!ta && !tb) {
        FDL_DMA_LAUNCH(false, false);
    } else if (!ta) {
        FDL_DMA_LAUNCH(false, true);
    } else if (!tb) {
        FDL_DMA_LAUNCH(true, false);
    } else {
        FDL_DMA_LAUNCH(true, true);
    }
#undef FDL_DMA_LAUNCH
    return hipGetLastError();
}

// Whether a hand-scheduled four-wave loop (CfgDma256W4, CfgDma128W4) runs
// this problem: K of at least 256, and each operand's extent (one batch)
// below 2 GiB, so the loop's 32-bit buffer offsets (lane part plus K-tile
// part) cannot wrap.
bool dma_w4_ok(const GemmParams& p, bool ta, bool tb) {
    constexpr int64_t kLimit = int64_t(1) << 31;
    const int64_t a_rows = ta ? p.K : p.M, a_cols = ta ? p.M : p.K;
    const int64_t b_rows = tb ? p.N : p.K, b_cols = tb ? p.K : p.N;
    const int64_t a_bytes = ((a_rows - 1) * p.lda + a_cols) * 4;
    const int64_t b_bytes = ((b_rows - 1) * p.ldb + b_cols) * 4;
    return p.K >= 256 && a_bytes < kLimit && b_bytes < kLimit;
}

// Launches the three-stage config One when the grid has at most one block
// per CU (256 CUs), else the two-stage Two, whose 64 KB of LDS lets two
// blocks share a CU.
template <class One, class Two>
hipError_t launch_dma_fit(const GemmParams& p, bool ta, bool tb, int nbatch, hipStream_t stream) {
    static_assert(One::BM == Two::BM && One::BN == Two::BN, "twins with the same tile");
    constexpr int64_t kCUs = 256;
    const int64_t blocks =
        (int64_t)((p.M + One::BM - 1) / One::BM) * ((p.N + One::BN - 1) / One::BN) * nbatch;
    return blocks <= kCUs ? launch_dma<One>(p, ta, tb, nbatch, stream)
                          : launch_dma<Two>(p, ta, tb, nbatch, stream);
}

template <int KW, int ITS = 4>
hipError_t launch_splitk32_kw(const GemmParams& p, bool ta, bool tb, bool va, bool vb,
                              int nbatch, hipStream_t stream) {
    if (!strides_fit32(p, nbatch)) {
        return launch_per_problem(p, nbatch, [&](const GemmParams& q) {
            return launch_splitk32_kw<KW, ITS>(q, ta, tb, va, vb, 1, stream);
        });
    }
    const int sa = nbatch > 1 ? (int)p.strideA : 0;
    const int sb = nbatch > 1 ? (int)p.strideB : 0;
    const int tiles_m = (p.M + 31) / 32;
    const int tiles_n = (p.N + 31) / 32;
    // K range per wave, a multiple of one super-chunk (8 * ITS steps), so only
    // the wave holding the end of K ever takes the guarded tail loads.
    constexpr int kSuper = 8 * ITS;
    int kchunk = (p.K + KW - 1) / KW;
    kchunk = std::max(kSuper, (kchunk + kSuper - 1) / kSuper * kSuper);
    const dim3 grid(tiles_m * tiles_n, nbatch);
    const dim3 block(KW * kWave);
    // VA is only used for k-contiguous A (not transposed), VB only for
    // k-contiguous B (transposed); normalise to avoid dead instantiations.
    va = va && !ta;
    vb = vb && tb;
    const int code = (ta ? 8 : 0) | (tb ? 4 : 0) | (va ? 2 : 0) | (vb ? 1 : 0);
#define FDL_SPLITK_CASE(C, TA_, TB_, VA_, VB_)                                          \
    case C:                                                                             \
        hipLaunchKernelGGL((sgemm_splitk32_kernel<KW, ITS, TA_, TB_, VA_, VB_>), grid,  \
                           block, 0, stream, p.A, p.B, p.lda, p.ldb, sa, sb, p.M, p.N,  \
                           p.K, kchunk, p);                                             \
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

// ---------------------------------------------------------------------------
// Grouped launches: up to four independent jobs in one grid, so that
// dependent chains of small kernels (the MLP step's backward pass) pay one
// launch for several jobs.  Every job body runs on 256 threads.
// ---------------------------------------------------------------------------
struct GroupDev {
    GemmParams p;
    int tiles_m, tiles_n, kchunk, blocks;
    const float* x;
    const float* x2;
    const int64_t* labels;
    float* out;
    float* out2;
    float* param;
    float lr;
    int64_t rows, cols;
};

constexpr int kGroupMaxJobs = 4;

struct GroupArgs {
    GroupDev d[kGroupMaxJobs];
};

constexpr int kGroupKW = 4;   // split-K waves of a grouped GEMM job (256 threads)
constexpr int kGroupITS = 8;  // 64 k of loads per wave in flight (MLP step 22.5 -> 21.9 us)

// Job 0's block count, and for a GEMM job 0 its shape and operand
// addresses: the grouped kernel takes them as leading scalar arguments,
// which arrive preloaded in SGPRs (the compiler preloads leading arguments
// that are not aggregates), so the first job's first loads wait for no
// scalar load of the GroupArgs aggregate.
struct GroupLead {
    const float* A;
    const float* B;
    int lda, ldb, M, N, K, tiles_m, tiles_n, kchunk, blocks;
};

template <bool TA, bool TB, bool VA, bool VB>
struct JobGemm {
    static __device__ __forceinline__ void run(const GroupDev& a, int bid) {
        splitk32_body<kGroupKW, kGroupITS, TA, TB, VA, VB>(a.p, a.tiles_m, a.tiles_n, a.kchunk,
                                                           bid, a.blocks, 0);
    }
    // As job 0: the lead's fields in place of the aggregate's.
    static __device__ __forceinline__ void run_first(const GroupLead& l, const GroupDev& a,
                                                     int bid) {
        GemmParams p = a.p;
        p.A = l.A;
        p.B = l.B;
        p.lda = l.lda;
        p.ldb = l.ldb;
        p.M = l.M;
        p.N = l.N;
        p.K = l.K;
        splitk32_body<kGroupKW, kGroupITS, TA, TB, VA, VB, true>(p, l.tiles_m, l.tiles_n,
                                                                 l.kchunk, bid, l.blocks, 0);
    }
};

// A kGemm16 job: four waves of split K, two 16-k groups of loads in flight
// per register buffer (MLP step with all four of a wave's groups at once:
// 16.36 -> 16.29 us per step; one group per buffer: 16.35 us).
constexpr int kGroupITS16 = 2;
template <bool TA, bool TB, bool VA, bool VB>
struct JobGemm16 {
    static __device__ __forceinline__ void run(const GroupDev& a, int bid) {
        splitk16_body<kGroupKW, kGroupITS16, TA, TB, VA, VB>(a.p, a.tiles_m, a.tiles_n,
                                                             a.kchunk, bid, a.blocks, 0);
    }
};

struct JobColsumSgd {
    static __device__ __forceinline__ void run(const GroupDev& a, int bid) {
        colsum_body(a.x, a.out, a.param, a.lr, a.rows, a.cols, bid);
    }
    static __device__ __forceinline__ void run_first(const GroupLead&, const GroupDev& a,
                                                     int bid) {
        run(a, bid);
    }
};

struct JobSgd {
    static __device__ __forceinline__ void run(const GroupDev& a, int bid) {
        sgd_body(a.param, a.x, a.lr, a.rows, bid, a.blocks);
    }
};

struct JobXentFinalize {
    static __device__ __forceinline__ void run(const GroupDev& a, int) {
        xent_finalize_body(a.x, (int)a.rows, (int)a.cols, a.out2, a.out, a.param, a.lr);
    }
};

// Two blocks: block 0 the loss, block 1 db and the bias step.
struct JobHeadFinalize {
    static __device__ __forceinline__ void run(const GroupDev& a, int bid) {
        if (a.cols <= 16) {
            head_finalize_body<16>(bid, a.x, a.x2, a.labels, a.rows, a.cols, a.out2, a.out,
                                   a.param, a.lr);
        } else {
            head_finalize_body<kColsumCols>(bid, a.x, a.x2, a.labels, a.rows, a.cols, a.out2,
                                            a.out, a.param, a.lr);
        }
    }
};

// Block `bid` of the grid runs job I if it falls in that job's range, else
// the next job with the index rebased.
template <int I, class J, class... Rest>
__device__ __forceinline__ void group_dispatch(const GroupArgs& a, int bid) {
    if constexpr (sizeof...(Rest) == 0) {
        J::run(a.d[I], bid);
    } else {
        if (bid < a.d[I].blocks) {
            J::run(a.d[I], bid);
        } else {
            group_dispatch<I + 1, Rest...>(a, bid - a.d[I].blocks);
        }
    }
}

template <class J0, class... Rest>
__global__ void __launch_bounds__(kGroupKW * kWave)
sgemm_group_kernel(const float* __restrict__ A0, const float* __restrict__ B0, int lda0,
                   int ldb0, int M0, int N0, int K0, int tiles_m0, int tiles_n0, int kchunk0,
                   int blocks0, GroupArgs a) {
    static_assert(sizeof...(Rest) >= 1 && sizeof...(Rest) < kGroupMaxJobs, "2 to 4 jobs");
    const int bid = blockIdx.x;
    if (bid < blocks0) {
        const GroupLead lead{A0, B0, lda0, ldb0, M0, N0, K0, tiles_m0, tiles_n0, kchunk0,
                             blocks0};
        J0::run_first(lead, a.d[0], bid);
    } else {
        group_dispatch<1, Rest...>(a, bid - blocks0);
    }
}

template <int KW, int ITS = 1>
hipError_t launch_splitk16_kw(const GemmParams& p, bool ta, bool tb, bool va, bool vb,
                              int nbatch, hipStream_t stream) {
    if (!strides_fit32(p, nbatch)) {
        return launch_per_problem(p, nbatch, [&](const GemmParams& q) {
            return launch_splitk16_kw<KW, ITS>(q, ta, tb, va, vb, 1, stream);
        });
    }
    const int sa = nbatch > 1 ? (int)p.strideA : 0;
    const int sb = nbatch > 1 ? (int)p.strideB : 0;
    const int tiles_m = (p.M + 15) / 16;
    const int tiles_n = (p.N + 15) / 16;
    constexpr int kSuper = 16 * ITS;
    int kchunk = (p.K + KW - 1) / KW;
    kchunk = std::max(kSuper, (kchunk + kSuper - 1) / kSuper * kSuper);
    const dim3 grid(tiles_m * tiles_n, nbatch);
    const dim3 block(KW * kWave);
    va = va && !ta;
    vb = vb && tb;
    const int code = (ta ? 8 : 0) | (tb ? 4 : 0) | (va ? 2 : 0) | (vb ? 1 : 0);
#define FDL_SPLITK16_CASE(C, TA_, TB_, VA_, VB_)                                        \
    case C:                                                                             \
        hipLaunchKernelGGL((sgemm_splitk16_kernel<KW, ITS, TA_, TB_, VA_, VB_>), grid,  \
                           block, 0, stream, p.A, p.B, p.lda, p.ldb, sa, sb, p.M, p.N,  \
                           p.K, kchunk, p);                                             \
        break;
    switch (code) {
        FDL_SPLITK16_CASE(0, false, false, false, false)
        FDL_SPLITK16_CASE(2, false, false, true, false)
        FDL_SPLITK16_CASE(4, false, true, false, false)
        FDL_SPLITK16_CASE(5, false, true, false, true)
        FDL_SPLITK16_CASE(6, false, true, true, false)
        FDL_SPLITK16_CASE(7, false, true, true, true)
        FDL_SPLITK16_CASE(8, true, false, false, false)
        FDL_SPLITK16_CASE(12, true, true, false, false)
        FDL_SPLITK16_CASE(13, true, true, false, true)
        default:
            return hipErrorInvalidValue;
    }
#undef FDL_SPLITK16_CASE
    return hipGetLastError();
}

// Waves per block by K (measured on the MLP-step shapes: 16 waves from
// K = 512, 8 from 128, else 4; one group in flight per buffer).
hipError_t launch_splitk16(const GemmParams& p, bool ta, bool tb, bool va, bool vb,
                           int nbatch, hipStream_t stream) {
    // NN with 16-byte rows and 64 k per wave: the LDS-staged form (its
    // 32-bit copy offsets span 16 rows of A and 64 rows of B).
    if (!ta && !tb && va && vb && p.K > 768 && p.K <= 1024 && p.lda < (int64_t(1) << 24) &&
        p.ldb < (int64_t(1) << 22)) {
        const dim3 grid(((p.M + 15) / 16) * ((p.N + 15) / 16), nbatch);
        const int waves = (p.K + 63) / 64;  // 13 to 16
        hipLaunchKernelGGL((sgemm_splitk16_lds_kernel<16, 64>), grid, dim3(waves * kWave), 0,
                           stream, p.A, p.B, p.strideA, p.strideB, (int)p.lda, (int)p.ldb, p.M,
                           p.N, p.K, p);
        return hipGetLastError();
    }
    if (p.K >= 512) return launch_splitk16_kw<16, 1>(p, ta, tb, va, vb, nbatch, stream);
    if (p.K >= 128) return launch_splitk16_kw<8, 1>(p, ta, tb, va, vb, nbatch, stream);
    return launch_splitk16_kw<4, 1>(p, ta, tb, va, vb, nbatch, stream);
}

// More waves per block for longer K, so each wave's range stays short
// (about 32-64 steps: one or two super-chunks of loads).
hipError_t launch_splitk32(const GemmParams& p, bool ta, bool tb, bool va, bool vb,
                           int nbatch, hipStream_t stream) {
    if (p.K >= 512) return launch_splitk32_kw<16, 2>(p, ta, tb, va, vb, nbatch, stream);
    if (p.K >= 128) return launch_splitk32_kw<8, 2>(p, ta, tb, va, vb, nbatch, stream);
    return launch_splitk32_kw<4, 2>(p, ta, tb, va, vb, nbatch, stream);
}

template <int MR, int STRIP, int NT, int UNR>
hipError_t launch_skinny_cfg(const GemmParams& p, bool ta, bool vb, int nbatch,
                             hipStream_t stream) {
    if (!strides_fit32(p, nbatch)) {
        return launch_per_problem(p, nbatch, [&](const GemmParams& q) {
            return launch_skinny_cfg<MR, STRIP, NT, UNR>(q, ta, vb, 1, stream);
        });
    }
    const int sa = nbatch > 1 ? (int)p.strideA : 0;
    const int sb = nbatch > 1 ? (int)p.strideB : 0;
    const int strips = (p.N + STRIP - 1) / STRIP;
    const dim3 grid(strips, nbatch);
    const dim3 block(NT);
#define FDL_SKINNY_LAUNCH(TA_, VB_)                                                         \
    hipLaunchKernelGGL((sgemm_skinny_kernel<MR, TA_, VB_, STRIP, NT, UNR>), grid, block, 0, \
                       stream, p.A, p.B, p.lda, p.ldb, sa, sb, p.M, p.N, p.K, strips, p)
    if (ta) {
        if (vb) FDL_SKINNY_LAUNCH(true, true);
        else FDL_SKINNY_LAUNCH(true, false);
    } else {
        if (vb) FDL_SKINNY_LAUNCH(false, true);
        else FDL_SKINNY_LAUNCH(false, false);
    }
#undef FDL_SKINNY_LAUNCH
    return hipGetLastError();
}

// 16-column strips, 256 threads; 8 B rows in flight per lane for M == 1,
// 512 threads with 8 rows in flight for larger M (measured on K = N = 4096).
template <int MR>
hipError_t launch_skinny_mr(const GemmParams& p, bool ta, bool vb, int nbatch,
                            hipStream_t stream) {
    if (MR == 1) return launch_skinny_cfg<MR, 16, 256, 8>(p, ta, vb, nbatch, stream);
    return launch_skinny_cfg<MR, 16, 512, 8>(p, ta, vb, nbatch, stream);
}

hipError_t launch_skinny(const GemmParams& p, bool ta, bool vb, int nbatch,
                         hipStream_t stream) {
    if (p.M <= 1) return launch_skinny_mr<1>(p, ta, vb, nbatch, stream);
    if (p.M <= 2) return launch_skinny_mr<2>(p, ta, vb, nbatch, stream);
    if (p.M <= 4) return launch_skinny_mr<4>(p, ta, vb, nbatch, stream);
    return launch_skinny_mr<8>(p, ta, vb, nbatch, stream);
}

template <int MR>
hipError_t launch_skinny_split_mr(const GemmParams& p, bool ta, const SkinnySplit& s,
                                  float* part, hipStream_t stream) {
    constexpr int UNR = 4;
    const dim3 grid1(s.bands * s.slices);
    const dim3 block1(kSplitWaves * kWave);
    const int tiles = s.bands * s.slices;
    if (ta) {
        hipLaunchKernelGGL((sgemm_skinny_part_kernel<MR, true, UNR>), grid1, block1, 0, stream,
                           p.A, p.B, part, (int)p.lda, (int)p.ldb, p.M, p.N, p.K, s.slices,
                           s.rows, tiles);
    } else {
        hipLaunchKernelGGL((sgemm_skinny_part_kernel<MR, false, UNR>), grid1, block1, 0, stream,
                           p.A, p.B, part, (int)p.lda, (int)p.ldb, p.M, p.N, p.K, s.slices,
                           s.rows, tiles);
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const dim3 grid2(s.bands, p.M);
    if (s.slices <= 16) {
        hipLaunchKernelGGL((sgemm_skinny_sum_kernel<MR, 16>), grid2, dim3(kSplitBand), 0, stream,
                           part, s.slices, p.N, p);
    } else if (s.slices <= 32) {
        hipLaunchKernelGGL((sgemm_skinny_sum_kernel<MR, 32>), grid2, dim3(kSplitBand), 0, stream,
                           part, s.slices, p.N, p);
    } else {
        hipLaunchKernelGGL((sgemm_skinny_sum_kernel<MR, kSplitMaxSlices>), grid2,
                           dim3(kSplitBand), 0, stream, part, s.slices, p.N, p);
    }
    return hipGetLastError();
}

hipError_t launch_skinny_split(const GemmParams& p, bool ta, const SkinnySplit& s,
                               float* part, hipStream_t stream) {
    switch (s.mr) {
        case 1: return launch_skinny_split_mr<1>(p, ta, s, part, stream);
        case 2: return launch_skinny_split_mr<2>(p, ta, s, part, stream);
        case 4: return launch_skinny_split_mr<4>(p, ta, s, part, stream);
        default: return launch_skinny_split_mr<8>(p, ta, s, part, stream);
    }
}

constexpr int kMaxGridY = 65535;

// Production tile configurations (BM, BN, BK, WM, WN, PAD, waves per SIMD).
using CfgTiled128 = TileCfg<128, 128, 16, 64, 64, 4, 1>;
using CfgTiled64 = TileCfg<64, 64, 16, 32, 32, 4, 1>;
// Tiled256 reads LDS fragments two k pairs at a time, the next chunk's reads
// issued ahead of the current chunk's MFMAs (measured +3-4% over whole-tile
// reads at 4096^3 and 8192^3).
using CfgTiled256 = TileCfg<256, 256, 16, 128, 64, 4, 1, 0, 2, 1, 1>;
using CfgTiled256x128 = TileCfg<256, 128, 16, 64, 64, 4, 1>;
using CfgTiled128W8 = TileCfg<128, 128, 16, 32, 64, 4, 1>;
// Direct-to-LDS configurations: two stages with the cross-tile pipeline and
// interleaved fragment reads (4096^3: 1.00-1.05 ms; 8192^3: 7.78 ms, 141
// TFLOP/s).  The 128x128 tile runs two blocks per CU and wins where 256x256
// tiles would leave CUs idle (2048^3: 0.161 vs 0.178 ms for Tiled128W8;
// 4000x3000x2048: 0.45 vs 0.54 ms for the 256x256 tile).
using CfgDma256 = DmaCfg<256, 256, 16, 128, 64, 2, 1, 1>;
// The same tile as four waves of 128x128 (one per SIMD, 256 accumulators in
// AGPRs) with three stages and the hand-scheduled steady-state loop of
// dma_loops.inc: problems with K >= 256 whose operands span less than 2 GiB
// (the loop's copies use 32-bit buffer offsets).  4096^3 NN: 945 -> 904-918
// us; results bit-identical to CfgDma256 (each output adds the same products
// in the same order).
using CfgDma256W4 = DmaCfg<256, 256, 16, 128, 128, 3, 1, 1, 1, 4, 1, 1>;
using CfgDma128 = DmaCfg<128, 128, 32, 64, 64, 2, 1, 1>;
// The same tile with three stages and the hand-scheduled loop of
// dma_loops.inc (96 KB of LDS: one block per CU), where the eight-wave
// 128x128 tile would run (2048^3 NN: 130.7 -> 118-120 us).
using CfgDma128W4 = DmaCfg<128, 128, 32, 64, 64, 3, 1, 1, 1, 4, 1, 1>;
// 64x64x64: mid-size problems whose 128x128 tiles cannot fill the GPU.  Two
// sets of four 32x32 waves split each K-tile's k-groups, so one block per CU
// still runs two waves per SIMD (1024^3: 24.3 vs 25.9 us with one set, and
// 42 us for the split-K kernel).
using CfgDma64 = DmaCfg<64, 64, 64, 32, 32, 2, 1, 1, 2>;
// Its three-stage twin, for grids of at most one block per CU: each tile's
// copies are spread over all four of its k-groups instead of the one after
// the barrier (96 KB of LDS, so one block per CU).
using CfgDma64S3 = DmaCfg<64, 64, 64, 32, 32, 3, 1, 1, 2>;
// Four waves of 32x32 (one per SIMD) with the hand-scheduled loop of
// dma_loops.inc, where the three-stage twin would run and K >= 256.
using CfgDma64W4 = DmaCfg<64, 64, 64, 32, 32, 3, 1, 1, 1, 4, 1, 1>;
// 128x128x64 with eight waves of 64x32 and 128 KB of LDS (one block per CU):
// two waves per SIMD where the GPU holds about one 128x128 tile per CU
// (2048^3: 131 vs 136.5 us for Dma128 in the same run).
using CfgDma128W8 = DmaCfg<128, 128, 64, 64, 32, 2, 1, 1>;
// The same tiles with 4-byte copies: any K, any leading dimension, any
// 4-byte-aligned pointer, at 2-3% below their 16-byte twins (1023^3: 26.5 us
// against 44 us for split-K; 4095^3: 1.11 ms).
using CfgDma64U = DmaCfg<64, 64, 64, 32, 32, 2, 1, 1, 2, 1>;
using CfgDma64US3 = DmaCfg<64, 64, 64, 32, 32, 3, 1, 1, 2, 1>;  // 1023^3: 24.1 -> 23.5 us
// 64x64x16 with four stages: every 16-deep K-tile of a short-K problem is
// copied at once and each is multiplied as soon as it lands, so a block's
// MFMAs overlap the arrival of its later tiles (the C4 batch, K = 64).
using CfgDma64S = DmaCfg<64, 64, 16, 32, 32, 4, 0, 1>;
// 96x32x64 with 4-byte copies and four k-group sets of three 32x32 waves
// (twelve waves, three per SIMD): three quarters of a 64x64 tile's work, for
// problems whose 64x64 tiles leave many CUs idle (777^3: 225 tiles instead
// of 169 on 256 CUs).  Its 32-wide operand's 2048 copy units do not divide
// over the 768 lanes; the surplus copies repeat the stage's last one.  Three
// stages, so each tile's eleven copies per lane are spread over both of its
// k-groups (777^3: 18.1 -> 17.4 us).
using CfgDma96x32U = DmaCfg<96, 32, 64, 32, 32, 3, 1, 1, 4, 1>;
using CfgDma128W8U = DmaCfg<128, 128, 64, 64, 32, 2, 1, 1, 1, 1>;

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

// The direct-to-LDS rows were fitted to back-to-back times of 26 NN, TN and
// NT problems from 1024^3 to 6144x6144x2048 and K from 64 to 4096 (the
// model's pick within 2.4% of the fastest direct-to-LDS tile on 23 of them,
// within 9% on the rest).
constexpr TileModel kTileModels[] = {
    {GemmKernel::Dma256, 256, 256, 1, 8, {0, 0.50f, 0.84f, 0.84f, 0.84f, 0.84f, 0.84f, 0.84f, 0.84f}},
    {GemmKernel::Dma128, 128, 128, 2, 4, {0, 0.75f, 0.83f, 0.83f, 0.83f, 0.83f, 0.83f, 0.83f, 0.83f}},
    {GemmKernel::Dma64, 64, 64, 2, 8, {0, 0.57f, 0.57f, 0.57f, 0.90f, 0.90f, 0.90f, 0.90f, 0.90f}},
    {GemmKernel::Dma128W8, 128, 128, 1, 8, {0, 0.78f, 0.78f, 0.78f, 0.78f, 0.78f, 0.78f, 0.78f, 0.78f}},
    {GemmKernel::Dma64U, 64, 64, 2, 8, {0, 0.553f, 0.553f, 0.67f, 0.67f, 0.67f, 0.67f, 0.67f, 0.67f}},
    {GemmKernel::Dma128W8U, 128, 128, 1, 8, {0, 0.757f, 0.757f, 0.757f, 0.757f, 0.757f, 0.757f, 0.757f, 0.757f}},
    // Measured at 777^3 (17.8 us for 225 tiles) against Dma64U (20.6 us for 169).
    {GemmKernel::Dma96x32U, 96, 32, 1, 12, {0, 0.48f, 0.48f, 0.48f, 0.48f, 0.48f, 0.48f, 0.48f, 0.48f}},
    {GemmKernel::Tiled256, 256, 256, 1, 8, {0, 0.50f, 0.79f, 0.79f, 0.79f, 0.79f, 0.79f, 0.79f, 0.79f}},
    {GemmKernel::Tiled256x128, 256, 128, 2, 8, {0, 0.45f, 0.70f, 0.74f, 0.79f, 0.79f, 0.79f, 0.79f, 0.79f}},
    {GemmKernel::Tiled128, 128, 128, 3, 4, {0, 0.565f, 0.66f, 0.71f, 0.71f, 0.71f, 0.71f, 0.71f, 0.71f}},
    {GemmKernel::Tiled128W8, 128, 128, 3, 8, {0, 0.45f, 0.63f, 0.68f, 0.72f, 0.74f, 0.75f, 0.75f, 0.75f}},
    {GemmKernel::Tiled64, 64, 64, 8, 4, {0, 0.30f, 0.45f, 0.52f, 0.60f, 0.63f, 0.65f, 0.67f, 0.68f}},
};

// Where the four-wave hand-scheduled form runs (NN, dma_w4_ok), Dma256 and
// Dma128W8 are faster than their rows above say (4096^3: 0.95; 2048^3 and
// 6144x6144x2048: 0.93).
constexpr float kW4Eff256 = 0.95f;
constexpr float kW4Eff128 = 0.93f;

// Each round of co-resident blocks also pays a fixed cost (its first
// copies' round trip and its stores), about 1 us, here in the same unit as
// the work: FMAs at one CU's fp32 MFMA rate (128 per clock at 2.4 GHz).  It
// matters only for short K (4096x4096x192: the 256x256 tile at 56 us against
// 68 us for the 64x64 tile's eight rounds).
constexpr double kRoundCost = 3.07e5;

double predicted_time(const TileModel& t, int M, int N, int K, int64_t batch) {
    constexpr int64_t kCUs = 256;
    const int64_t tiles = (int64_t)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * batch;
    const int64_t per_cu = (tiles + kCUs - 1) / kCUs;
    const double work = (double)t.bm * t.bn * K;
    const int64_t full = per_cu / t.slots;
    const int64_t rest = per_cu % t.slots;
    auto round_cost = [&](int64_t blocks) {
        const int w = (int)std::min<int64_t>(8, std::max<int64_t>(1, blocks * t.waves / 4));
        return (double)blocks * work / t.eff[w] + kRoundCost;
    };
    double time = (double)full * round_cost(t.slots);
    if (rest) time += round_cost(rest);
    return time;
}

// Direct-to-LDS kernels with 4-byte copies (any shape).
bool is_dma4(GemmKernel k) {
    return k == GemmKernel::Dma64U || k == GemmKernel::Dma128W8U || k == GemmKernel::Dma96x32U;
}

bool is_dma(GemmKernel k) {
    return k == GemmKernel::Dma256 || k == GemmKernel::Dma128 || k == GemmKernel::Dma64 ||
           k == GemmKernel::Dma128W8 || k == GemmKernel::Dma64S || is_dma4(k);
}

// Largest leading dimension of the 4-byte-copy kernels: a copy's 32-bit
// lane offset spans up to 32 rows of 4-byte elements.
constexpr int64_t kDma4MaxLd = int64_t(1) << 24;
// Largest leading dimension of the 16-byte-copy kernels: a wave's copies span
// up to 64 rows, so its 32-bit lane offsets stay below 2^31 bytes.
constexpr int64_t kDmaMaxLd = int64_t(1) << 22;

// Shape part of a direct-to-LDS kernel's contract (pointers not needed).
bool dma_shape_ok(GemmKernel k, const GemmParams& p, bool transA, bool transB) {
    if (is_dma4(k)) return p.K >= 1 && p.lda <= kDma4MaxLd && p.ldb <= kDma4MaxLd;
    const int64_t a_contig = transA ? p.M : p.K;
    const int64_t b_contig = transB ? p.K : p.N;
    return p.K >= 4 && p.K % 4 == 0 && a_contig % 4 == 0 && b_contig % 4 == 0 &&
           p.lda % 4 == 0 && p.ldb % 4 == 0 && p.lda <= kDmaMaxLd && p.ldb <= kDmaMaxLd;
}

inline bool aligned4(const void* ptr) {
    return (reinterpret_cast<uintptr_t>(ptr) & 3u) == 0;
}

}  // namespace

bool dma_supported(GemmKernel k, const GemmParams& p, bool transA, bool transB,
                   int64_t batch) {
    if (!is_dma(k) || !dma_shape_ok(k, p, transA, transB)) return false;
    if (is_dma4(k)) return aligned4(p.A) && aligned4(p.B);
    return vec_ok(p.A, transA ? p.M : p.K, p.lda, p.strideA, batch) &&
           vec_ok(p.B, transB ? p.K : p.N, p.ldb, p.strideB, batch);
}

const char* kernel_name(GemmKernel k) {
    switch (k) {
        case GemmKernel::Tiled128: return "tiled128";
        case GemmKernel::Tiled64: return "tiled64";
        case GemmKernel::SplitK32: return "splitk32";
        case GemmKernel::Skinny: return "skinny";
        case GemmKernel::Tiled256: return "tiled256";
        case GemmKernel::Tiled256x128: return "tiled256x128";
        case GemmKernel::Tiled128W8: return "tiled128w8";
        case GemmKernel::SplitK16: return "splitk16";
        case GemmKernel::Dma256: return "dma256";
        case GemmKernel::Dma128: return "dma128";
        case GemmKernel::Dma64: return "dma64";
        case GemmKernel::Dma128W8: return "dma128w8";
        case GemmKernel::Dma64U: return "dma64u";
        case GemmKernel::Dma128W8U: return "dma128w8u";
        case GemmKernel::Dma64S: return "dma64s";
        case GemmKernel::Dma96x32U: return "dma96x32u";
        case GemmKernel::Auto: return "auto";
    }
    return "unknown";
}

GemmKernel choose_kernel(const GemmParams& p, bool transA, bool transB,
                         int64_t batch) {
    // Skinny M: one streaming pass over B on the VALU beats an MFMA tile
    // that would be at most 8/32 occupied.
    if (p.M <= 8 && !transB && p.N >= 64) return GemmKernel::Skinny;
    const int64_t t64 = (int64_t)((p.M + 63) / 64) * ((p.N + 63) / 64) * batch;
    constexpr int64_t kCUs = 256;
    // Too few 64x64 tiles to occupy the GPU: split K over the waves of a
    // block instead, with 16x16 output tiles when 32x32 ones would leave most
    // CUs idle.  With K >= 256 the 64x64 direct-to-LDS tile wins from ~160
    // tiles (777^3: 21.9 vs 25.2 us; 1024^3: 22 vs 42 us).  Short K (64 to
    // 255) needs a full GPU of 64x64 tiles (the C4 batch of 64 128x128x64
    // problems: 5.0-5.2 vs 6.1-6.2 us for split-K; 1024x1024x128: 6.5 vs 8.4
    // us).  Below 128 tiles of 128x128, split-K still wins when the 64x64
    // tile count passes a multiple of the CU count by only a few tiles, whose
    // second round would run nearly empty (1000x1100x96 NT, 288 tiles:
    // split-K 8.7 vs 9.1 us).
    const int64_t t128 = (int64_t)((p.M + 127) / 128) * ((p.N + 127) / 128) * batch;
    const int64_t rem = t64 % kCUs;
    const bool long_k = p.K >= 256;
    if (p.K < 64 || t64 < (long_k ? 160 : kCUs) ||
        (!long_k && t128 < 128 && rem > 0 && rem < 64)) {
        const int64_t t32 = (int64_t)((p.M + 31) / 32) * ((p.N + 31) / 32) * batch;
        return t32 < 128 ? GemmKernel::SplitK16 : GemmKernel::SplitK32;
    }
    // The direct-to-LDS tiles compete where their shape contract holds (the
    // 4-byte-copy ones almost always); the register-staged tiles only when
    // none does.  launch_sgemm moves a 16-byte choice to its 4-byte twin
    // when the pointers turn out misaligned.
    GemmKernel best = GemmKernel::Tiled64;
    double best_time = 0.0;
    bool first = true;
    for (int pass = 0; pass < 2 && first; ++pass) {
        for (const TileModel& t : kTileModels) {
            if (is_dma(t.kernel) != (pass == 0)) continue;
            if (is_dma(t.kernel) && !dma_shape_ok(t.kernel, p, transA, transB)) continue;
            TileModel tw = t;
            if ((t.kernel == GemmKernel::Dma256 || t.kernel == GemmKernel::Dma128W8) &&
                dma_w4_ok(p, transA, transB)) {
                for (int w = 1; w <= 8; ++w)
                    tw.eff[w] = t.kernel == GemmKernel::Dma256 ? kW4Eff256 : kW4Eff128;
                tw.eff[1] = t.kernel == GemmKernel::Dma256 ? t.eff[1] : kW4Eff128;
            }
            const double tm = predicted_time(tw, p.M, p.N, p.K, batch);
            if (first || tm < best_time * 0.99) {  // ties keep the earlier (larger) tile
                best = t.kernel;
                best_time = tm;
                first = false;
            }
        }
    }
    // K of at most 128: every 16-deep K-tile in flight at once beats one or
    // two 64-deep tiles that must land whole (the C4 batch, 64 x 128x128x64:
    // 5.5 vs 6.0 us from HBM).
    if (best == GemmKernel::Dma64 && p.K <= 128) best = GemmKernel::Dma64S;
    return best;
}

SkinnySplit skinny_split_plan(const GemmParams& p, bool transA, bool transB, int64_t batch) {
    SkinnySplit s;
    if (batch != 1 || choose_kernel(p, transA, transB, batch) != GemmKernel::Skinny) return s;
    if (p.M < 1 || p.N % 4 != 0 || p.K < 1) return s;
    // (the partial pass takes its leading dimensions as 32-bit arguments)
    if (p.lda > INT32_MAX || p.ldb > INT32_MAX) return s;
    // The second pass costs about 3 us.  It pays when each strip of the
    // single pass is long (K >= 4096: 1.1x at N = 4096, 1.35x at N = 1024,
    // 3.2x at N = 1024, K = 16384) or B is large (N = 16384, K = 1024:
    // 1.2x), not for shorter K at moderate size (N = 4096, K = 1024: 0.75x;
    // N = 1024, K = 2048: 0.94x).
    if (p.K < 4096 && (int64_t)p.N * p.K < kSplitMinElems) return s;
    // About two rounds of the 256 CUs (1.6 at M <= 2), slices of at least 64
    // rows.  Blocks per launch, measured at K = N = 4096 (graph-timed, both
    // passes): M = 1 14.6-14.8 us at 512 blocks, 14.3-14.4 at 416, 15.1 at
    // 400, 14.8 at 432 and at 448, 14.5-14.7 at 384, 15.3 at 320, 17.1 at
    // 1024; M = 2 14.8-15.0 / 14.6 at 512 / 416; M = 4 and 8 were best at
    // 512 (16.0 / 16.4 and 17.8 / 18.4 against 384).  The rate depends on
    // where the slices start in B (see the 4 MiB rule below) as much as on
    // the block count.
    const int64_t bands = (p.N + kSplitBand - 1) / kSplitBand;
    const int64_t target = p.M <= 2 ? 416 : 512;
    int64_t slices = std::min<int64_t>(kSplitMaxSlices, (target + bands - 1) / bands);
    int64_t rows = (p.K + slices - 1) / slices;
    rows = std::max<int64_t>(64, (rows + 7) / 8 * 8);
    // Slices that start a multiple of 4 MiB of B apart read the same HBM
    // channels at the same time: 8 more rows per slice (the last slice
    // shorter) spread them.  Graph-timed, M = 8: N = 4096, K = 8192 (256-row
    // slices, 4 MiB apart) 37.7 -> 28.4 us; N = 16384, K = 1024 19.0 ->
    // 16.4 us; N = 16384, K = 4096 58.0 -> 50.9 us; C5a (2 MiB apart)
    // unchanged, and shifting 2 MiB strides as well made it slower (17.8 ->
    // 18.6 us: the short last slice).  The workspace-size query has no ldb
    // (0 here) and plans without the shift, which never takes fewer slices,
    // so the size it returns covers the call's.
    if (p.ldb > 0 && (rows * p.ldb * (int64_t)sizeof(float)) % (int64_t(4) << 20) == 0) {
        rows += 8;
    }
    slices = (p.K + rows - 1) / rows;
    if (slices < 2 || bands * slices > (1 << 22)) return s;
    s.mr = p.M <= 1 ? 1 : p.M <= 2 ? 2 : p.M <= 4 ? 4 : 8;
    s.bands = (int)bands;
    s.slices = (int)slices;
    s.rows = (int)rows;
    s.bytes = (size_t)bands * slices * s.mr * kSplitBand * sizeof(float);
    return s;
}

namespace {

GroupDev group_dev(const GroupJob& j) {
    GroupDev d{};
    d.p = j.p;
    d.x = j.x;
    d.x2 = j.x2;
    d.labels = j.labels;
    d.out = j.out;
    d.out2 = j.out2;
    d.param = j.param;
    d.lr = j.lr;
    d.rows = j.rows;
    d.cols = j.cols;
    switch (j.kind) {
        case GroupJob::kGemm: {
            d.tiles_m = (j.p.M + 31) / 32;
            d.tiles_n = (j.p.N + 31) / 32;
            constexpr int kSuper = 8 * kGroupITS;
            int kchunk = (j.p.K + kGroupKW - 1) / kGroupKW;
            d.kchunk = std::max(kSuper, (kchunk + kSuper - 1) / kSuper * kSuper);
            d.blocks = d.tiles_m * d.tiles_n;
            break;
        }
        case GroupJob::kGemm16: {
            d.tiles_m = (j.p.M + 15) / 16;
            d.tiles_n = (j.p.N + 15) / 16;
            constexpr int kSuper = 16 * kGroupITS16;
            int kchunk = (j.p.K + kGroupKW - 1) / kGroupKW;
            d.kchunk = std::max(kSuper, (kchunk + kSuper - 1) / kSuper * kSuper);
            d.blocks = d.tiles_m * d.tiles_n;
            break;
        }
        case GroupJob::kColsumSgd:
            d.blocks = (int)((j.cols + kColsumCols - 1) / kColsumCols);
            break;
        case GroupJob::kSgd:
            d.blocks = (int)std::min<int64_t>((j.rows + 4 * 256 - 1) / (4 * 256), 1024);
            break;
        case GroupJob::kXentFinalize:
            d.blocks = 1;
            break;
        case GroupJob::kHeadFinalize:
            d.blocks = 2;
            break;
    }
    return d;
}

template <class... J>
hipError_t launch_group_of(const GroupArgs& a, hipStream_t stream) {
    int blocks = 0;
    for (int i = 0; i < (int)sizeof...(J); ++i) blocks += a.d[i].blocks;
    const GroupDev& d0 = a.d[0];
    hipLaunchKernelGGL((sgemm_group_kernel<J...>), dim3(blocks), dim3(kGroupKW * kWave), 0,
                       stream, d0.p.A, d0.p.B, (int)d0.p.lda, (int)d0.p.ldb, d0.p.M, d0.p.N,
                       d0.p.K, d0.tiles_m, d0.tiles_n, d0.kchunk, d0.blocks, a);
    return hipGetLastError();
}

// The NT GEMM job with the vector flags launch_sgemm would derive for it (A
// and B both k-contiguous), followed by the jobs Rest.
template <class... Rest>
hipError_t launch_nt_first(const GroupJob& j0, const GroupArgs& a, hipStream_t stream) {
    const bool va = vec_ok(j0.p.A, j0.p.K, j0.p.lda, j0.p.strideA, 1);
    const bool vb = vec_ok(j0.p.B, j0.p.K, j0.p.ldb, j0.p.strideB, 1);
    if (va && vb) return launch_group_of<JobGemm<false, true, true, true>, Rest...>(a, stream);
    if (va) return launch_group_of<JobGemm<false, true, true, false>, Rest...>(a, stream);
    if (vb) return launch_group_of<JobGemm<false, true, false, true>, Rest...>(a, stream);
    return launch_group_of<JobGemm<false, true, false, false>, Rest...>(a, stream);
}

}  // namespace

hipError_t launch_group(const GroupJob* jobs, int n, hipStream_t stream) {
    if (n < 2 || n > kGroupMaxJobs) return hipErrorInvalidValue;
    GroupArgs a{};
    for (int i = 0; i < n; ++i) {
        const GroupJob& j = jobs[i];
        if ((j.kind == GroupJob::kGemm || j.kind == GroupJob::kGemm16) &&
            (j.p.M <= 0 || j.p.N <= 0 || j.p.K <= 0)) {
            return hipErrorInvalidValue;
        }
        // (the first job's leading dimensions travel as 32-bit kernel arguments)
        if (i == 0 && (j.p.lda > INT32_MAX || j.p.ldb > INT32_MAX)) return hipErrorInvalidValue;
        if (j.kind == GroupJob::kHeadFinalize &&
            (j.rows <= 0 || j.cols <= 0 || j.cols > kColsumCols)) {
            return hipErrorInvalidValue;
        }
        a.d[i] = group_dev(j);
    }
    auto is_nt = [&](int i) {
        return jobs[i].kind == GroupJob::kGemm && !jobs[i].ta && jobs[i].tb;
    };
    auto is_tn = [&](int i) {
        return jobs[i].kind == GroupJob::kGemm && jobs[i].ta && !jobs[i].tb;
    };
    auto is = [&](int i, GroupJob::Kind k) { return jobs[i].kind == k; };
    auto is_tn16 = [&](int i) {
        return jobs[i].kind == GroupJob::kGemm16 && jobs[i].ta && !jobs[i].tb;
    };
    using TN = JobGemm<true, false, false, false>;
    using TN16 = JobGemm16<true, false, false, false>;
    if (n == 2) {
        if (is_nt(0) && is_tn(1)) return launch_nt_first<TN>(jobs[0], a, stream);
        if (is_nt(0) && is(1, GroupJob::kColsumSgd)) {
            return launch_nt_first<JobColsumSgd>(jobs[0], a, stream);
        }
        if (is_tn(0) && is(1, GroupJob::kSgd)) return launch_group_of<TN, JobSgd>(a, stream);
    } else if (n == 3) {
        if (is(0, GroupJob::kColsumSgd) && is_tn(1) && is(2, GroupJob::kXentFinalize)) {
            return launch_group_of<JobColsumSgd, TN, JobXentFinalize>(a, stream);
        }
    } else {
        if (is_nt(0) && is(1, GroupJob::kColsumSgd) && is_tn(2) &&
            is(3, GroupJob::kXentFinalize)) {
            return launch_nt_first<JobColsumSgd, TN, JobXentFinalize>(jobs[0], a, stream);
        }
        if (is_tn(0) && is(1, GroupJob::kColsumSgd) && is_tn(2) &&
            is(3, GroupJob::kHeadFinalize)) {
            return launch_group_of<TN, JobColsumSgd, TN, JobHeadFinalize>(a, stream);
        }
        if (is_tn(0) && is(1, GroupJob::kColsumSgd) && is_tn16(2) &&
            is(3, GroupJob::kHeadFinalize)) {
            return launch_group_of<TN, JobColsumSgd, TN16, JobHeadFinalize>(a, stream);
        }
    }
    return hipErrorInvalidValue;
}

hipError_t launch_sgemm(const GemmParams& p0, bool transA, bool transB,
                        int64_t batch, GemmKernel kernel, hipStream_t stream,
                        float* workspace, size_t workspace_bytes) {
    if (batch <= 0 || p0.M <= 0 || p0.N <= 0) return hipSuccess;
    const bool automatic = kernel == GemmKernel::Auto;
    if (automatic) kernel = choose_kernel(p0, transA, transB, batch);
    if (kernel == GemmKernel::Skinny && (transB || p0.M > 8)) return hipErrorInvalidValue;
    if (is_dma(kernel) && !dma_supported(kernel, p0, transA, transB, batch)) {
        if (!automatic) return hipErrorInvalidValue;
        // Misaligned pointers: the 4-byte-copy tile, else the register-staged one.
        const GemmKernel u = (kernel == GemmKernel::Dma64 || kernel == GemmKernel::Dma64S)
                                 ? GemmKernel::Dma64U
                                 : GemmKernel::Dma128W8U;
        if (!is_dma4(kernel) && dma_supported(u, p0, transA, transB, batch)) {
            kernel = u;
        } else {
            kernel = kernel == GemmKernel::Dma256     ? GemmKernel::Tiled256
                     : kernel == GemmKernel::Dma128   ? GemmKernel::Tiled128
                     : kernel == GemmKernel::Dma128W8 ? GemmKernel::Tiled128W8
                     : kernel == GemmKernel::Dma128W8U ? GemmKernel::Tiled128W8
                                                      : GemmKernel::Tiled64;
        }
    }

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
            case GemmKernel::SplitK16:
                err = launch_splitk16(p, transA, transB, va, vb, nb, stream);
                break;
            case GemmKernel::Skinny: {
                const SkinnySplit split = skinny_split_plan(p0, transA, transB, batch);
                if (workspace != nullptr && split.slices > 0 && vb &&
                    workspace_bytes >= split.bytes) {
                    err = launch_skinny_split(p, transA, split, workspace, stream);
                } else {
                    err = launch_skinny(p, transA, vb, nb, stream);
                }
                break;
            }
            case GemmKernel::Dma256:
                err = dma_w4_ok(p, transA, transB)
                          ? launch_dma<CfgDma256W4>(p, transA, transB, nb, stream)
                          : launch_dma<CfgDma256>(p, transA, transB, nb, stream);
                break;
            case GemmKernel::Dma128:
                err = launch_dma<CfgDma128>(p, transA, transB, nb, stream);
                break;
            case GemmKernel::Dma64:
                err = dma_w4_ok(p, transA, transB)
                          ? launch_dma_fit<CfgDma64W4, CfgDma64>(p, transA, transB, nb, stream)
                          : launch_dma_fit<CfgDma64S3, CfgDma64>(p, transA, transB, nb, stream);
                break;
            case GemmKernel::Dma128W8:
                err = dma_w4_ok(p, transA, transB)
                          ? launch_dma<CfgDma128W4>(p, transA, transB, nb, stream)
                          : launch_dma<CfgDma128W8>(p, transA, transB, nb, stream);
                break;
            case GemmKernel::Dma64U:
                err = launch_dma_fit<CfgDma64US3, CfgDma64U>(p, transA, transB, nb, stream);
                break;
            case GemmKernel::Dma128W8U:
                err = launch_dma<CfgDma128W8U>(p, transA, transB, nb, stream);
                break;
            case GemmKernel::Dma64S:
                err = launch_dma<CfgDma64S>(p, transA, transB, nb, stream);
                break;
            case GemmKernel::Dma96x32U:
                err = launch_dma<CfgDma96x32U>(p, transA, transB, nb, stream);
                break;
            default:
                return hipErrorInvalidValue;
        }
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

}  // namespace fdl
