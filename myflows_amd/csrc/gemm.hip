// FP32 GEMM engine on the CDNA4 matrix cores: C(M x N) = op(A) op(B) (+ bias) (activation),
// row-major, with op(X) = X or X^T chosen per operand. The MFMA main loop, the LDS layouts, the
// XCD-grouped tile order and the epilogue are in gemm_core.h; this file holds the dense operand
// loads, the split-K reduction, the tile catalogue and the planner.
//
// The third grid dimension has two uses:
//   * split-K (GemmParams::split = 1): z selects the K slice [z * k_chunk, min(K, (z+1) * k_chunk))
//     and writes its partial product to C + z * c_batch; split_reduce then sums the slices in a fixed
//     order in FP64;
//   * batches (split = 0): z is an independent problem at A + z * a_batch, B + z * b_batch,
//     C + z * c_batch.
// Every output element is produced by one wave in one fixed order, so results are bitwise
// reproducible run to run.
#include <algorithm>

#include "common.h"
#include "gemm_core.h"

namespace mfh {
namespace {

constexpr const GemmTile* TILES = GEMM_TILES;
constexpr int NUM_TILES = GEMM_TILE_COUNT;
constexpr int MAX_SLICES = 128;   // slices of the automatic planner
constexpr int MIN_CHUNK = 256;    // smallest K slice the automatic planner makes

// Explicit GEMM plan codes, with the reference's arithmetic (ops/cuda_native/native_cublas.cpp:
// 1264-1269, 1335-1344; native.py:298-309):
//   NAMED_BASE + n * NAMED_SLICES + (slices - 1), slices <= 32: the reference's named tile n
//     (128x128, 128x64, 256x32, 64x128, 32x256), run on this catalogue's tile for the same role
//     (NAMED_TILE_OF: general, N <= 64, N <= 32, M <= 64, M <= 32 outputs);
//   EXTENDED_BASE + i * EXTENDED_SLICES + (slices - 1), slices <= 128: tile i of this catalogue
//     (mfh_gemm_tile_info), as the reference's extended codes index its own catalogue.
constexpr int NAMED_BASE = 16, NAMED_SLICES = 32, NAMED_COUNT = 5;
constexpr int EXTENDED_BASE = 1024, EXTENDED_SLICES = 128;
constexpr int NAMED_TILE_OF[NAMED_COUNT] = {0, 1, 4, 2, 5};
// The engine's k pairing: the two terms of an MFMA are 8 apart in sub-stages of 16 k, for every
// tile (the 32-deep stages of the 256x256 tile included), so that every one-group tile adds an
// output's K terms in one order.
constexpr int GEMM_PAIR = 8;

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_mfma_kernel(GemmParams p) {
    using S = MfmaShape<BM, BN, BK, WM, WN, TA, TB, 4, 4, GEMM_PAIR>;
    __shared__ __attribute__((aligned(16))) float smem[2 * S::STAGE];

    int tile_m, tile_n, z;
    tile_of_workgroup(tile_m, tile_n, z);
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int wm0 = (wave / S::WGN) * WM, wn0 = (wave % S::WGN) * WN;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const float* __restrict__ A = p.A + (p.split ? 0 : z * p.a_batch);
    const float* __restrict__ B = p.B + (p.split ? 0 : z * p.b_batch);
    float* __restrict__ C = p.C + z * p.c_batch;
    const int k_begin = p.split ? z * p.k_chunk : 0;
    const int k_end = p.split ? min(p.K, k_begin + p.k_chunk) : p.K;
    const int M = p.M, N = p.N;

    // A tile: rows = m (k-contiguous) or k (mn-contiguous); likewise B.
    TileLoader<TA ? BK : BM, TA ? BM : BK, S::THREADS, VA> la;
    TileLoader<TB ? BN : BK, TB ? BK : BN, S::THREADS, VB> lb;
    auto fetch = [&](int kt) {
        if constexpr (TA) la.load(A, p.lda, kt, k_end, m0, M, tid);
        else la.load(A, p.lda, m0, M, kt, k_end, tid);
        if constexpr (TB) lb.load(B, p.ldb, n0, N, kt, k_end, tid);
        else lb.load(B, p.ldb, kt, k_end, n0, N, tid);
    };
    auto store = [&](float* a_lds, float* b_lds) {
        la.template store<S::LDA_S>(a_lds, tid);
        lb.template store<S::LDB_S>(b_lds, tid);
    };

    v16f acc[S::TM][S::TN];
    zero_acc<S>(acc);
    // The 16-deep tiles run two or more workgroups per CU and gain from a raised priority over
    // the MFMAs; the 32-deep 256x256 tile (one workgroup per CU) from an early store of the next
    // stage.
    constexpr int ORDER = BK >= 32 ? STAGE_EARLY_STORE : STAGE_PRIORITY;
    mfma_k_loop<S, ORDER>(smem, k_begin, k_end, fetch, store, acc, wm0, wn0, lane);
    store_acc<S>(p, C, acc, m0, n0, wm0, wn0, lane);
}

// A tile whose K range is shared by KG groups of (BM/WM) x (BN/WN) waves (KG x the waves of
// gemm_mfma_kernel for the same tile, so that a small output still has several waves per SIMD):
// group g runs the stages [g * per, (g + 1) * per) of the workgroup's K range (per = the stage
// count over KG, rounded up; stages past the end read zeros, which add exact zeros, so that every
// group passes the same barriers) on its own double-buffered LDS stage with its global reads two
// stages ahead, each output's terms in one FP32 chain; the groups' sums are then added in group
// order ((g0 + g1) + g2) + ... through LDS, and group 0 writes the tile. Fixed order: bitwise
// reproducible run to run (a grouped tile sums in another order than the one-group tiles).
template <int BM, int BN, int BK, int WM, int WN, int KG, bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64 * KG) void gemm_grouped_kernel(GemmParams p) {
    using S = MfmaShape<BM, BN, BK, WM, WN, TA, TB, 4, 4, GEMM_PAIR>;
    constexpr int PARTIAL = S::THREADS * 16 * S::TM * S::TN;  // floats of one group's accumulators
    static_assert((KG - 1) * PARTIAL <= KG * 2 * S::STAGE, "the group sums fit in the stage buffers");
    __shared__ __attribute__((aligned(16))) float smem[KG * 2 * S::STAGE];

    int tile_m, tile_n, z;
    tile_of_workgroup(tile_m, tile_n, z);
    const int group = threadIdx.x / S::THREADS, tid = threadIdx.x % S::THREADS;
    const int wave = tid / 64, lane = tid % 64;
    const int wm0 = (wave / S::WGN) * WM, wn0 = (wave % S::WGN) * WN;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const float* __restrict__ A = p.A + (p.split ? 0 : z * p.a_batch);
    const float* __restrict__ B = p.B + (p.split ? 0 : z * p.b_batch);
    float* __restrict__ C = p.C + z * p.c_batch;
    const int k_begin = p.split ? z * p.k_chunk : 0;
    const int k_end = p.split ? min(p.K, k_begin + p.k_chunk) : p.K;
    const int M = p.M, N = p.N;
    const int per = ((k_end - k_begin + BK - 1) / BK + KG - 1) / KG;  // stages of every group
    const int g_begin = k_begin + group * per * BK;

    using LoadA = TileLoader<TA ? BK : BM, TA ? BM : BK, S::THREADS, VA>;
    using LoadB = TileLoader<TB ? BN : BK, TB ? BK : BN, S::THREADS, VB>;
    LoadA la[2];
    LoadB lb[2];
    // Every load is bounded by k_end (reads past it give zeros), the ahead loop's fetches past the
    // end included.
    auto fetch = [&](auto slot, int kt) {
        constexpr int T = decltype(slot)::value;
        if constexpr (TA) la[T].load(A, p.lda, kt, k_end, m0, M, tid);
        else la[T].load(A, p.lda, m0, M, kt, k_end, tid);
        if constexpr (TB) lb[T].load(B, p.ldb, n0, N, kt, k_end, tid);
        else lb[T].load(B, p.ldb, kt, k_end, n0, N, tid);
    };
    auto store = [&](auto slot, float* a_lds, float* b_lds) {
        constexpr int T = decltype(slot)::value;
        la[T].template store<S::LDA_S>(a_lds, tid);
        lb[T].template store<S::LDB_S>(b_lds, tid);
    };

    v16f acc[S::TM][S::TN];
    zero_acc<S>(acc);
    // NN products store the next stage half-way through a stage's MFMAs (1024^3 27.5 -> 26.7 us on
    // MI355X), a transposed A after them (the dW form 43.3 against 44.0 us).
    constexpr int ORDER = TA || TB ? STAGE_PLAIN : STAGE_MID_STORE;
    mfma_k_loop_ahead<S, ORDER>(smem + group * 2 * S::STAGE, g_begin, g_begin + per * BK, fetch, store, acc, wm0,
                                wn0, lane);
    // The loop ends with a barrier: every group is done with the stage buffers.
    if (group > 0) {
        float* mine = smem + (group - 1) * PARTIAL + tid;
#pragma unroll
        for (int i = 0; i < S::TM; ++i)
#pragma unroll
            for (int j = 0; j < S::TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) mine[((i * S::TN + j) * 16 + r) * S::THREADS] = acc[i][j][r];
    }
    __syncthreads();
    if (group > 0) return;
#pragma unroll
    for (int g = 1; g < KG; ++g) {
        const float* theirs = smem + (g - 1) * PARTIAL + tid;
#pragma unroll
        for (int i = 0; i < S::TM; ++i)
#pragma unroll
            for (int j = 0; j < S::TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] += theirs[((i * S::TN + j) * 16 + r) * S::THREADS];
    }
    store_acc<S>(p, C, acc, m0, n0, wm0, wn0, lane);
}

// C = act((float)(((0.0 + p0) + p1) + ... + p[S-1]) [+ bias]) with the FP64 sum in slice order,
// the bias (per column or per row) added in FP32 after the rounding, stored dense (row * ldc + col)
// or segmented like the GEMM's own epilogue (C = C + that when p.accumulate).
__device__ __forceinline__ void finish_output(const GemmParams& p, float* C, long long i, double s) {
    const int row = static_cast<int>(i / p.N), col = static_cast<int>(i % p.N);
    float v = static_cast<float>(s);
    if (p.bias_mode == BIAS_COLUMN) v += p.bias[col];
    else if (p.bias_mode == BIAS_ROW) v += p.bias[row];
    if (p.residual) v = v + p.residual[output_offset(p, row, col)];
    write_output(p, C, row, col, activate(v, p.act, p.alpha));
}

constexpr int REDUCE_AHEAD = 8;  // slices loaded before they are added

// The rows riding on a split-K reduction (GemmParams::row_out): wave w of the launch finishes row
// w. Lane l adds slices l, l + 64, ... in order, then a fixed butterfly adds the lanes (FP64
// throughout), so the result does not depend on timing.
__device__ __forceinline__ void finish_row(const GemmParams& p, long long t) {
    const long long row = t / 64;
    if (row >= p.row_count) return;  // uniform over the wave
    const int lane = static_cast<int>(t % 64);
    double s = 0.0;
    for (int z = lane; z < p.row_slices; z += 64) s += p.row_partial[static_cast<long long>(z) * p.row_count + row];
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) s += __shfl_xor(s, offset, 64);
    if (lane == 0) p.row_out[row] = static_cast<float>(s);
}

// One thread per output; the loads of REDUCE_AHEAD slices are issued before their additions, which
// still run one at a time in slice order.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ partial, float* __restrict__ C,
                                                           GemmParams p, int slices) {
    raise_wave_priority();
    const long long i = blockIdx.x * 256LL + threadIdx.x, total = static_cast<long long>(p.M) * p.N;
    if (p.row_out) finish_row(p, i);
    if (i >= total) return;
    double s = 0.0;
    int z = 0;
    for (; z + REDUCE_AHEAD <= slices; z += REDUCE_AHEAD) {
        float part[REDUCE_AHEAD];
#pragma unroll
        for (int u = 0; u < REDUCE_AHEAD; ++u) part[u] = partial[(z + u) * total + i];
#pragma unroll
        for (int u = 0; u < REDUCE_AHEAD; ++u) s += static_cast<double>(part[u]);
    }
    for (; z < slices; ++z) s += static_cast<double>(partial[z * total + i]);
    finish_output(p, C, i, s);
}

// Four adjacent outputs per thread with 16-byte loads (M * N % 4 == 0, aligned partials); the same
// slice-order FP64 sums as split_reduce_kernel.
__global__ __launch_bounds__(256) void split_reduce_vec4_kernel(const float* __restrict__ partial,
                                                                float* __restrict__ C, GemmParams p, int slices) {
    raise_wave_priority();
    const long long q = blockIdx.x * 256LL + threadIdx.x, total = static_cast<long long>(p.M) * p.N;
    if (p.row_out) finish_row(p, q);
    if (q * 4 >= total) return;
    const float4* quads = reinterpret_cast<const float4*>(partial);
    const long long stride = total / 4;
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    int z = 0;
    for (; z + REDUCE_AHEAD <= slices; z += REDUCE_AHEAD) {
        float4 part[REDUCE_AHEAD];
#pragma unroll
        for (int u = 0; u < REDUCE_AHEAD; ++u) part[u] = quads[(z + u) * stride + q];
#pragma unroll
        for (int u = 0; u < REDUCE_AHEAD; ++u) {
            s0 += static_cast<double>(part[u].x);
            s1 += static_cast<double>(part[u].y);
            s2 += static_cast<double>(part[u].z);
            s3 += static_cast<double>(part[u].w);
        }
    }
    for (; z < slices; ++z) {
        const float4 part = quads[z * stride + q];
        s0 += static_cast<double>(part.x);
        s1 += static_cast<double>(part.y);
        s2 += static_cast<double>(part.z);
        s3 += static_cast<double>(part.w);
    }
    finish_output(p, C, q * 4, s0);
    finish_output(p, C, q * 4 + 1, s1);
    finish_output(p, C, q * 4 + 2, s2);
    finish_output(p, C, q * 4 + 3, s3);
}

// Many slices over few outputs (a dW product split over the pixels): thread (q, g) of a block of
// GROUP_QUADS x REDUCE_GROUPS threads sums the slices [g * per, (g + 1) * per) of outputs 4q .. 4q+3 in
// slice order in FP64; the group sums are then added in group order. The order is fixed, so the
// result does not depend on timing (it is the slice-order sum regrouped, not its bits).
constexpr int REDUCE_GROUPS = 8, GROUP_QUADS = 32;
__global__ __launch_bounds__(REDUCE_GROUPS* GROUP_QUADS) void split_reduce_grouped_kernel(
    const float* __restrict__ partial, float* __restrict__ C, GemmParams p, int slices) {
    __shared__ double group_sum[REDUCE_GROUPS][GROUP_QUADS][4];
    const long long t = blockIdx.x * static_cast<long long>(REDUCE_GROUPS * GROUP_QUADS) + threadIdx.x;
    if (p.row_out) finish_row(p, t);
    const int g = threadIdx.x / GROUP_QUADS, qi = threadIdx.x % GROUP_QUADS;
    const long long q = blockIdx.x * static_cast<long long>(GROUP_QUADS) + qi, total = static_cast<long long>(p.M) * p.N;
    const long long stride = total / 4;
    const int per = (slices + REDUCE_GROUPS - 1) / REDUCE_GROUPS;
    const int z0 = g * per, z1 = min(slices, z0 + per);
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    if (q < stride) {
        const float4* quads = reinterpret_cast<const float4*>(partial);
        int z = z0;
        for (; z + REDUCE_AHEAD <= z1; z += REDUCE_AHEAD) {
            float4 part[REDUCE_AHEAD];
#pragma unroll
            for (int u = 0; u < REDUCE_AHEAD; ++u) part[u] = quads[(z + u) * stride + q];
#pragma unroll
            for (int u = 0; u < REDUCE_AHEAD; ++u) {
                s0 += static_cast<double>(part[u].x);
                s1 += static_cast<double>(part[u].y);
                s2 += static_cast<double>(part[u].z);
                s3 += static_cast<double>(part[u].w);
            }
        }
        for (; z < z1; ++z) {
            const float4 part = quads[z * stride + q];
            s0 += static_cast<double>(part.x);
            s1 += static_cast<double>(part.y);
            s2 += static_cast<double>(part.z);
            s3 += static_cast<double>(part.w);
        }
    }
    group_sum[g][qi][0] = s0;
    group_sum[g][qi][1] = s1;
    group_sum[g][qi][2] = s2;
    group_sum[g][qi][3] = s3;
    __syncthreads();
    if (g != 0 || q >= stride) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        double sum = group_sum[0][qi][r];
#pragma unroll
        for (int h = 1; h < REDUCE_GROUPS; ++h) sum += group_sum[h][qi][r];
        finish_output(p, C, q * 4 + r, sum);
    }
}

using GemmFn = void (*)(GemmParams);
constexpr int VARIANTS = 16;  // 4 layouts (NN, NT, TN, TT) x float4 loads of A (yes/no) x of B

template <int T, bool TA, bool TB, bool VA, bool VB>
constexpr GemmFn kernel_of() {
    constexpr GemmTile t = TILES[T];
    if constexpr (t.kg > 1) return gemm_grouped_kernel<t.bm, t.bn, t.bk, t.wm, t.wn, t.kg, TA, TB, VA, VB>;
    else return gemm_mfma_kernel<t.bm, t.bn, t.bk, t.wm, t.wn, TA, TB, VA, VB>;
}

template <int T, bool TA, bool TB>
constexpr void fill_layout(GemmFn* slot) {
    slot[0] = kernel_of<T, TA, TB, false, false>();
    slot[1] = kernel_of<T, TA, TB, false, true>();
    slot[2] = kernel_of<T, TA, TB, true, false>();
    slot[3] = kernel_of<T, TA, TB, true, true>();
}

template <int T>
constexpr void fill_row(GemmFn (&row)[VARIANTS]) {
    fill_layout<T, false, false>(row + 0);
    fill_layout<T, false, true>(row + 4);
    fill_layout<T, true, false>(row + 8);
    fill_layout<T, true, true>(row + 12);
}

struct KernelTable {
    GemmFn fn[NUM_TILES][VARIANTS];
    KernelTable() {
        fill_row<0>(fn[0]);
        fill_row<1>(fn[1]);
        fill_row<2>(fn[2]);
        fill_row<3>(fn[3]);
        fill_row<4>(fn[4]);
        fill_row<5>(fn[5]);
        fill_row<6>(fn[6]);
        fill_row<7>(fn[7]);
        fill_row<8>(fn[8]);
        fill_row<9>(fn[9]);
    }
};
static_assert(NUM_TILES == 10, "KernelTable lists every tile");

const KernelTable& kernel_table() {
    static const KernelTable table;
    return table;
}

int threads_of(const GemmTile& t) { return (t.bm / t.wm) * (t.bn / t.wn) * 64 * t.kg; }

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15) == 0; }

// Planner model of one workgroup tile: relative MFMA efficiency once latency is hidden, and how many
// workgroups fit on a CU at once (registers and LDS). Fitted to a sweep of every tile and split on
// MI355X over the ResNet18 batch-64 GEMM shapes and 4096^3.
struct TileCost {
    double efficiency;
    int per_cu;
};
constexpr TileCost COST[NUM_TILES] = {
    {1.063, 3}, {0.95, 3}, {0.85, 4}, {0.935, 6}, {0.60, 6}, {0.60, 6}, {1.02, 2}, {1.02, 2}, {0.93, 3}, {1.07, 1},
};
constexpr double HIDING_HALF = 0.75;  // resident waves per SIMD at which half the latency is hidden
constexpr int SPLITS[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64, 96, 128};

// Estimated time of a plan in CU multiply-adds (a CU retires 128 FP32 multiply-adds per clock on
// its matrix cores): the busiest CU runs ceil(workgroups / CUs) tiles of BM * BN * chunk
// multiply-adds at the tile's efficiency, scaled by how much memory latency its resident waves hide
// (w / (w + HIDING_HALF) for w waves per SIMD). A split adds the partials' HBM round trip (written
// once, read once, about 2 KB per clock chip-wide, so 0.064 units per byte) and one more launch
// (about 5 us = 1.5e6 units).
double plan_cost(int tile, std::int64_t workgroups, int chunk, std::int64_t M, std::int64_t N, int slices) {
    const GemmTile& t = TILES[tile];
    const int cus = std::max(1, device_cu_count());
    const std::int64_t per_cu = (workgroups + cus - 1) / cus;
    const double waves_per_simd = static_cast<double>(std::min<std::int64_t>(per_cu, COST[tile].per_cu)) *
                                  ((t.bm / t.wm) * (t.bn / t.wn) * t.kg) / 4.0;
    const double hiding = waves_per_simd / (waves_per_simd + HIDING_HALF);
    double cost = static_cast<double>(per_cu) * t.bm * t.bn * chunk / (COST[tile].efficiency * hiding);
    if (slices > 1) cost += 0.064 * 4.0 * (2.0 * slices + 1.0) * static_cast<double>(M) * N + 1.5e6;
    return cost;
}

}  // namespace

int gemm_tile_count() { return NUM_TILES; }
const GemmTile& gemm_tile(int index) { return TILES[index]; }

// The plan of least estimated cost over every tile and (for a single problem) every split of K
// into slices of at least MIN_CHUNK: large outputs take large tiles; small outputs trade tile size
// and K slices for enough workgroups to fill the GPU.
GemmPlan gemm_auto_plan(int M, int N, int K, int batch, unsigned tiles) {
    GemmPlan best{0, 1, K};
    double best_cost = -1.0;
    for (int tile = 0; tile < NUM_TILES; ++tile) {
        if (!(tiles & (1u << tile))) continue;
        const GemmTile& t = TILES[tile];
        const std::int64_t tiles = static_cast<std::int64_t>(blocks_for(M, t.bm)) * blocks_for(N, t.bn) * batch;
        if (blocks_for(M, t.bm) > GRID_YZ_LIMIT) continue;
        const int max_split = batch > 1 ? 1 : std::max(1, std::min(MAX_SLICES, K / MIN_CHUNK));
        for (const int requested : SPLITS) {
            if (requested > max_split) break;
            const int chunk = static_cast<int>(((static_cast<std::int64_t>(K) + requested - 1) / requested + t.bk - 1) /
                                               t.bk * t.bk);
            const int slices = (K + chunk - 1) / chunk;
            if (slices > GRID_YZ_LIMIT) continue;
            const double cost = plan_cost(tile, tiles * slices, std::min(chunk, K), M, N, slices);
            if (best_cost < 0 || cost < best_cost) {
                best_cost = cost;
                best = GemmPlan{tile, slices, slices > 1 ? chunk : K};
            }
        }
    }
    return best;
}

bool gemm_engine_valid(int engine) {
    return engine == 1 || (engine >= NAMED_BASE && engine < NAMED_BASE + NAMED_COUNT * NAMED_SLICES) ||
           (engine >= EXTENDED_BASE && engine < EXTENDED_BASE + NUM_TILES * EXTENDED_SLICES);
}

int gemm_plan_from_engine(int engine, int M, int N, int K, GemmPlan* plan, int batch) {
    if (!gemm_engine_valid(engine)) return MFH_FAIL(ERR_ARG, "unknown GEMM engine or plan code");
    if (engine == 1) {
        *plan = gemm_auto_plan(M, N, K, batch);
        return OK;
    }
    const bool named = engine < EXTENDED_BASE;
    const int code = engine - (named ? NAMED_BASE : EXTENDED_BASE);
    const int per_tile = named ? NAMED_SLICES : EXTENDED_SLICES;
    const int tile = named ? NAMED_TILE_OF[code / per_tile] : code / per_tile, requested = code % per_tile + 1;
    const int bk = TILES[tile].bk;
    const std::int64_t rounded = ((static_cast<std::int64_t>(K) + requested - 1) / requested + bk - 1) / bk * bk;
    const int chunk = static_cast<int>(std::min<std::int64_t>(K, rounded));
    *plan = GemmPlan{tile, static_cast<int>((static_cast<std::int64_t>(K) + chunk - 1) / chunk), chunk};
    return OK;
}

std::int64_t gemm_workspace_floats(const GemmPlan& plan, int M, int N) {
    return plan.slices > 1 ? static_cast<std::int64_t>(plan.slices) * M * N : 0;
}


namespace {

GemmParams epilogue_params(const GemmEpilogue& e, int M, int N, int ldc) {
    GemmParams p{};
    p.M = M;
    p.N = N;
    p.ldc = ldc;
    p.bias = e.bias;
    p.bias_mode = e.bias_mode;
    p.act = e.act;
    p.alpha = e.alpha;
    p.segment = e.segment;
    if (e.segment > 0) p.segment_div = FastDiv(e.segment);
    p.segment_stride = e.segment_stride;
    p.taps = e.taps;
    if (e.taps > 0) p.taps_div = FastDiv(e.taps);
    p.accumulate = e.accumulate ? 1 : 0;
    p.residual = e.residual;
    p.lattice_w = e.lattice_w;
    if (e.lattice_w > 0) p.lattice_div = FastDiv(e.lattice_w);
    p.lattice_row = e.lattice_row;
    p.lattice_col = e.lattice_col;
    p.lattice_offset = e.lattice_offset;
    p.cell_h = e.cell_h;
    p.cell_w = e.cell_w;
    p.plane_h = e.plane_h;
    p.plane_w = e.plane_w;
    p.row_partial = e.row_partial;
    p.row_out = e.row_out;
    p.row_count = e.row_out ? e.row_count : 0;
    return p;
}

int launch_split_reduce(const float* partial, float* c, GemmParams p, int slices, hipStream_t stream) {
    const std::int64_t outputs = static_cast<std::int64_t>(p.M) * p.N;
    p.row_slices = slices;
    if (outputs % 4 == 0 && aligned16(partial)) {
        const std::int64_t threads = std::max<std::int64_t>(outputs / 4, 64LL * p.row_count);
        launch(split_reduce_vec4_kernel, blocks_for(threads, 256), 256, 0, stream, partial, c, p, slices);
        return MFH_CHECK_LAUNCH("split_reduce_vec4", stream);
    }
    const std::int64_t threads = std::max<std::int64_t>(outputs, 64LL * p.row_count);
    launch(split_reduce_kernel, blocks_for(threads, 256), 256, 0, stream, partial, c, p, slices);
    return MFH_CHECK_LAUNCH("split_reduce", stream);
}

}  // namespace

int split_reduce(const float* partial, float* c, int slices, int M, int N, int ldc, bool /*reference*/,
                 hipStream_t stream) {
    return launch_split_reduce(partial, c, epilogue_params(GemmEpilogue{}, M, N, ldc), slices, stream);
}

int split_reduce_grouped(const float* partial, float* c, const GemmEpilogue& e, int M, int N, int ldc, int slices,
                         hipStream_t stream) {
    GemmParams p = epilogue_params(e, M, N, ldc);
    p.row_slices = slices;
    const std::int64_t outputs = static_cast<std::int64_t>(M) * N;
    if (outputs % 4 != 0 || !aligned16(partial)) return launch_split_reduce(partial, c, p, slices, stream);
    const std::int64_t blocks = std::max<std::int64_t>(blocks_for(outputs / 4, GROUP_QUADS),
                                                       blocks_for(64LL * p.row_count, REDUCE_GROUPS * GROUP_QUADS));
    launch(split_reduce_grouped_kernel, blocks, REDUCE_GROUPS * GROUP_QUADS, 0, stream, partial, c, p, slices);
    return MFH_CHECK_LAUNCH("split_reduce_grouped", stream);
}

int split_reduce_epilogue(const float* partial, float* c, const GemmEpilogue& e, int M, int N, int ldc, int slices,
                          hipStream_t stream) {
    return launch_split_reduce(partial, c, epilogue_params(e, M, N, ldc), slices, stream);
}

namespace {

// Outputs with few columns (N <= SKINNY_N, a matrix-vector-like product such as a small fully
// connected layer): one wave per output row; lane l adds a[row][k] * b[k][n] for k = l, l + 64, ...
// in k order, then a fixed butterfly adds the lanes, so every output has one summation order. The
// MFMA tiles would leave all but N of their 32 or more columns idle and spend their time in
// prologue and epilogue.
constexpr int SKINNY_N = 8;
__global__ __launch_bounds__(256) void gemm_skinny_kernel(GemmParams p, int trans_a, int trans_b) {
    const int row = static_cast<int>(blockIdx.x) * 4 + static_cast<int>(threadIdx.x) / 64, lane = threadIdx.x % 64;
    if (row >= p.M) return;  // uniform over the wave
    float acc[SKINNY_N];
#pragma unroll
    for (int n = 0; n < SKINNY_N; ++n) acc[n] = 0.0f;
    for (int k = lane; k < p.K; k += 64) {
        const float a = trans_a ? p.A[static_cast<long long>(k) * p.lda + row] : p.A[static_cast<long long>(row) * p.lda + k];
#pragma unroll
        for (int n = 0; n < SKINNY_N; ++n)
            if (n < p.N)
                acc[n] += a * (trans_b ? p.B[static_cast<long long>(n) * p.ldb + k] : p.B[static_cast<long long>(k) * p.ldb + n]);
    }
#pragma unroll
    for (int n = 0; n < SKINNY_N; ++n)
#pragma unroll
        for (int offset = 32; offset > 0; offset >>= 1) acc[n] += __shfl_xor(acc[n], offset, 64);
    if (lane != 0) return;
#pragma unroll
    for (int n = 0; n < SKINNY_N; ++n) {
        if (n >= p.N) break;
        float v = acc[n];
        if (p.bias_mode == BIAS_COLUMN) v += p.bias[n];
        else if (p.bias_mode == BIAS_ROW) v += p.bias[row];
        write_output(p, p.C, row, n, activate(v, p.act, p.alpha));
    }
}

// Whether gemm_launch runs the problem on gemm_skinny_kernel.
bool takes_skinny(int engine, int batch, int N, const GemmEpilogue& e) {
    return engine == 1 && batch == 1 && N <= SKINNY_N && e.segment == 0 && e.taps == 0 && e.lattice_w == 0 &&
           !e.residual;
}

}  // namespace

std::int64_t gemm_launch_workspace(int engine, int M, int N, int K) {
    if (takes_skinny(engine, 1, N, GemmEpilogue{})) return 0;
    GemmPlan plan;
    if (gemm_plan_from_engine(engine, M, N, K, &plan) != OK) return -1;
    return gemm_workspace_floats(plan, M, N);
}

int gemm_launch(int engine, hipStream_t stream, const GemmOperands& o, const GemmEpilogue& e, float* workspace,
                std::int64_t workspace_floats) {
    const int M = o.M, N = o.N, K = o.K;
    if (takes_skinny(engine, o.batch, N, e)) {
        GemmParams p = epilogue_params(e, M, N, o.ldc);
        p.A = o.a;
        p.B = o.b;
        p.C = o.c;
        p.K = K;
        p.lda = o.lda;
        p.ldb = o.ldb;
        p.k_chunk = K;
        launch(gemm_skinny_kernel, blocks_for(M, 4), 256, 0, stream, p, o.trans_a ? 1 : 0, o.trans_b ? 1 : 0);
        return MFH_CHECK_LAUNCH("gemm_skinny", stream);
    }
    GemmPlan plan;
    MFH_TRY(gemm_plan_from_engine(engine, M, N, K, &plan, o.batch));
    if (o.batch > 1 || (plan.slices > 1 && (!workspace || workspace_floats < gemm_workspace_floats(plan, M, N))))
        plan = GemmPlan{plan.tile, 1, K};
    const bool split = plan.slices > 1;
    // float4 loads of an operand need its contiguous extent, its leading dimension, its batch stride
    // and its base pointer to be multiples of 4 floats / 16 bytes (K slices are multiples of BK).
    const bool vec_a = (o.trans_a ? M : K) % 4 == 0 && o.lda % 4 == 0 && o.a_batch % 4 == 0 && aligned16(o.a);
    const bool vec_b = (o.trans_b ? K : N) % 4 == 0 && o.ldb % 4 == 0 && o.b_batch % 4 == 0 && aligned16(o.b);
    const GemmTile& tile = TILES[plan.tile];
    const std::int64_t planes = split ? plan.slices : o.batch;
    const std::int64_t workgroups = static_cast<std::int64_t>(blocks_for(M, tile.bm)) * blocks_for(N, tile.bn) * planes;
    if (blocks_for(M, tile.bm) > GRID_YZ_LIMIT || planes > GRID_YZ_LIMIT || workgroups > INDEX_LIMIT)
        return MFH_FAIL(ERR_ARG, "GEMM grid exceeds the launch limits");
    GemmParams p = epilogue_params(e, M, N, o.ldc);
    p.A = o.a;
    p.B = o.b;
    p.K = K;
    p.lda = o.lda;
    p.ldb = o.ldb;
    p.a_batch = o.a_batch;
    p.b_batch = o.b_batch;
    if (split) {
        p.C = workspace;
        p.ldc = N;
        p.c_batch = static_cast<long long>(M) * N;
        p.split = 1;
        p.k_chunk = plan.k_chunk;
        p.bias = nullptr;
        p.bias_mode = BIAS_NONE;
        p.act = ACT_NONE;
        p.segment = 0;
        p.taps = 0;
        p.accumulate = 0;
        p.residual = nullptr;
    } else {
        p.C = o.c;
        p.c_batch = o.c_batch;
        p.split = 0;
        p.k_chunk = K;
    }
    const int layout = (o.trans_a ? 2 : 0) + (o.trans_b ? 1 : 0);  // NN, NT, TN, TT
    const GemmFn fn = kernel_table().fn[plan.tile][layout * 4 + (vec_a ? 2 : 0) + (vec_b ? 1 : 0)];
    const dim3 grid(blocks_for(N, tile.bn), blocks_for(M, tile.bm), static_cast<unsigned>(planes));
    launch(fn, grid, dim3(threads_of(tile)), 0, stream, p);
    MFH_TRY(MFH_CHECK_LAUNCH("gemm_mfma", stream));
    if (!split) return OK;
    return launch_split_reduce(workspace, o.c, epilogue_params(e, M, N, o.ldc), plan.slices, stream);
}

}  // namespace mfh
