// FP32 GEMM engine on the CDNA4 matrix cores: C(M x N) = op(A) op(B) (+ bias) (activation),
// row-major, with op(X) = X or X^T chosen per operand.
//
// Work decomposition. A workgroup computes a BM x BN tile of C with (BM/WM) x (BN/WN) wave64s; a
// wave owns a WM x WN sub-tile made of (WM/32) x (WN/32) accumulators of v_mfma_f32_32x32x2_f32
// (16 floats per lane each). The K range of the workgroup is consumed in BK-deep stages that are
// double buffered in LDS: the global loads of stage t+1 are in flight while the waves run the
// MFMAs of stage t, with one barrier per stage.
//
// LDS layout. Each operand tile is kept in LDS in the orientation it has in global memory, so the
// global->LDS copy is a straight (float4 when aligned) row copy with no transpose:
//   * "k-contiguous" operands (A when not transposed, B when transposed) live as [rows][BK + 4];
//   * "mn-contiguous" operands (A when transposed, B when not transposed) live as [BK][rows + 4].
// The +4 floats of padding keep 16-byte alignment and move successive rows to other banks.
//
// MFMA operand mapping. v_mfma_f32_32x32x2_f32 multiplies a 32x2 slice of A (lane l supplies
// A[l % 32][l / 32]) by a 2x32 slice of B (lane l supplies B[l / 32][l % 32]) and accumulates the
// 32x32 product; lane l holds output column l % 32, rows 8 * (r / 4) + 4 * (l / 32) + r % 4 in its
// register r. Which k a lane half (l / 32) feeds at each step is free as long as A and B agree, so
// half h consumes k = h * BK/2 + s for s = 0 .. BK/2 - 1: a k-contiguous operand then reads four
// consecutive k of its row with one 16-byte LDS load. Every tile uses the same BK and the same k
// mapping, so an unsplit product adds each output's K terms in the same order whatever the tile.
//
// Tile order. Workgroups are handed to the 8 XCDs round-robin by their linear id, and each XCD has
// its own L2. The kernel renumbers the workgroups so that XCD x receives one contiguous run of
// tiles, walked in groups of GROUP_M tile rows (column by column inside a group): the tiles an XCD
// runs at the same time share A row panels and B column panels in its L2.
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

namespace mfh {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

// Tile catalogue: block tile BM x BN, stage depth BK, wave tile WM x WN (multiples of 32).
constexpr GemmTile TILES[] = {
    {128, 128, 16, 64, 64},  // 0: general
    {256, 64, 16, 64, 64},   // 1: tall outputs, N <= 64
    {64, 128, 16, 32, 64},   // 2: short outputs, M <= 64
    {64, 64, 16, 32, 32},    // 3: small outputs
    {128, 32, 16, 32, 32},   // 4: N <= 32
    {32, 128, 16, 32, 32},   // 5: M <= 32
    {256, 128, 16, 64, 64},  // 6: large outputs, 8 waves
    {128, 256, 16, 64, 64},  // 7: large outputs, 8 waves
};
constexpr int NUM_TILES = sizeof(TILES) / sizeof(TILES[0]);
constexpr int PLAN_BASE = 16;     // engine codes >= PLAN_BASE name a tile and a slice count
constexpr int MAX_SLICES = 128;   // slices per explicit plan code
constexpr int MIN_CHUNK = 256;    // smallest K slice the automatic planner makes
constexpr int GROUP_M = 8;        // tile rows per group of the tile order
constexpr int XCDS = 8;           // accelerator complex dies of an MI355X

// A ROWS x COLS tile whose COLS dimension is contiguous in global memory (row stride ld), staged
// through registers: load() issues the global reads, store() writes them to LDS.
template <int ROWS, int COLS, int THREADS, bool VEC>
struct TileLoader {
    static constexpr int ELEMS = VEC ? ROWS * COLS / 4 : ROWS * COLS;
    static constexpr int PER_THREAD = (ELEMS + THREADS - 1) / THREADS;
    static constexpr int VCOLS = VEC ? COLS / 4 : COLS;
    float4 v[VEC ? PER_THREAD : 1];
    float s[VEC ? 1 : PER_THREAD];

    __device__ __forceinline__ void load(const float* __restrict__ base, int ld, int row0, int row_limit, int col0,
                                         int col_limit, int tid) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) {
            const int f = tid + i * THREADS;
            const int r = f / VCOLS, c = f % VCOLS;
            const int row = row0 + r;
            if constexpr (VEC) {
                const int col = col0 + c * 4;
                float4 value = make_float4(0.f, 0.f, 0.f, 0.f);
                if (f < ELEMS && row < row_limit && col < col_limit)
                    value = *reinterpret_cast<const float4*>(base + static_cast<long long>(row) * ld + col);
                v[i] = value;
            } else {
                const int col = col0 + c;
                float value = 0.f;
                if (f < ELEMS && row < row_limit && col < col_limit) value = base[static_cast<long long>(row) * ld + col];
                s[i] = value;
            }
        }
    }

    template <int LD>
    __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) {
            const int f = tid + i * THREADS;
            if (f >= ELEMS) continue;
            const int r = f / VCOLS, c = f % VCOLS;
            if constexpr (VEC) *reinterpret_cast<float4*>(lds + r * LD + c * 4) = v[i];
            else lds[r * LD + c] = s[i];
        }
    }
};

__device__ __forceinline__ float activate(float v, int act, float alpha) {
    if (act == ACT_RELU) return v < 0.0f ? 0.0f : v;  // NaN stays NaN
    if (act == ACT_LEAKY_RELU) return v > 0.0f ? v : alpha * v;
    return v;
}

// Where output (row, col) of problem z lives.
__device__ __forceinline__ long long output_offset(const GemmParams& p, int row, int col) {
    if (p.segment) {
        int within;
        const int segment = p.segment_div.divmod(col, within);
        return segment * p.segment_stride + static_cast<long long>(row) * p.ldc + within;
    }
    return static_cast<long long>(row) * p.ldc + col;
}

// (tile row, tile column, z) of this workgroup in the XCD-grouped order described above.
__device__ __forceinline__ void tile_of_workgroup(int& tile_m, int& tile_n, int& z) {
    const int gx = gridDim.x, gy = gridDim.y;
    const int plane = gx * gy;
    const int total = plane * gridDim.z;
    const int linear = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const int xcd = linear % XCDS, position = linear / XCDS;
    const int base = total / XCDS, extra = total % XCDS;
    const int logical = xcd * base + min(xcd, extra) + position;
    z = logical / plane;
    const int t = logical - z * plane;
    const int group_span = GROUP_M * gx;
    const int first_m = (t / group_span) * GROUP_M;
    const int rows = min(gy - first_m, GROUP_M);
    const int in_group = t - (t / group_span) * group_span;
    tile_m = first_m + in_group % rows;
    tile_n = in_group / rows;
}

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_mfma_kernel(GemmParams p) {
    constexpr int WGN = BN / WN, THREADS = (BM / WM) * WGN * 64;
    constexpr int TM = WM / 32, TN = WN / 32, HALF = BK / 2;
    static_assert(BK % 8 == 0, "each lane half consumes groups of four k");
    // LDS row lengths (floats) of the A and B tiles in their global orientation.
    constexpr int LDA_S = TA ? BM + 4 : BK + 4;
    constexpr int LDB_S = TB ? BK + 4 : BN + 4;
    constexpr int A_SIZE = TA ? BK * LDA_S : BM * LDA_S;
    constexpr int B_SIZE = TB ? BN * LDB_S : BK * LDB_S;
    __shared__ __attribute__((aligned(16))) float smem[2 * (A_SIZE + B_SIZE)];

    int tile_m, tile_n, z;
    tile_of_workgroup(tile_m, tile_n, z);
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int lm = lane % 32, h = lane / 32;
    const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    const float* __restrict__ A = p.A + (p.split ? 0 : z * p.a_batch);
    const float* __restrict__ B = p.B + (p.split ? 0 : z * p.b_batch);
    float* __restrict__ C = p.C + z * p.c_batch;
    const int k_begin = p.split ? z * p.k_chunk : 0;
    const int k_end = p.split ? min(p.K, k_begin + p.k_chunk) : p.K;
    const int M = p.M, N = p.N;

    // A tile: rows = m (k-contiguous) or k (mn-contiguous); likewise B.
    TileLoader<TA ? BK : BM, TA ? BM : BK, THREADS, VA> la;
    TileLoader<TB ? BN : BK, TB ? BK : BN, THREADS, VB> lb;
    auto fetch = [&](int kt) {
        if constexpr (TA) la.load(A, p.lda, kt, k_end, m0, M, tid);
        else la.load(A, p.lda, m0, M, kt, k_end, tid);
        if constexpr (TB) lb.load(B, p.ldb, n0, N, kt, k_end, tid);
        else lb.load(B, p.ldb, kt, k_end, n0, N, tid);
    };
    auto stage = [&](int buf) {
        la.template store<LDA_S>(smem + buf * (A_SIZE + B_SIZE), tid);
        lb.template store<LDB_S>(smem + buf * (A_SIZE + B_SIZE) + A_SIZE, tid);
    };

    v16f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int stages = k_end > k_begin ? (k_end - k_begin + BK - 1) / BK : 0;
    if (stages > 0) {
        fetch(k_begin);
        stage(0);
    }
    __syncthreads();
    for (int t = 0; t < stages; ++t) {
        const bool more = t + 1 < stages;
        if (more) fetch(k_begin + (t + 1) * BK);
        const float* As = smem + (t & 1) * (A_SIZE + B_SIZE);
        const float* Bs = As + A_SIZE;
#pragma unroll
        for (int kk = 0; kk < HALF; kk += 4) {
            const int k = h * HALF + kk;
            float4 a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int m = wm0 + i * 32 + lm;
                if constexpr (TA)
                    a[i] = make_float4(As[k * LDA_S + m], As[(k + 1) * LDA_S + m], As[(k + 2) * LDA_S + m],
                                       As[(k + 3) * LDA_S + m]);
                else a[i] = *reinterpret_cast<const float4*>(As + m * LDA_S + k);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = wn0 + j * 32 + lm;
                if constexpr (TB) b[j] = *reinterpret_cast<const float4*>(Bs + n * LDB_S + k);
                else
                    b[j] = make_float4(Bs[k * LDB_S + n], Bs[(k + 1) * LDB_S + n], Bs[(k + 2) * LDB_S + n],
                                       Bs[(k + 3) * LDB_S + n]);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
                }
        }
        if (more) stage((t + 1) & 1);
        __syncthreads();
    }

    // Epilogue: bias (per output column or per output row), the activation, then the store.
    const float* __restrict__ bias = p.bias;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn0 + j * 32 + lm;
        if (col >= N) continue;
        const float col_bias = p.bias_mode == BIAS_COLUMN ? bias[col] : 0.f;
        const long long col_offset = output_offset(p, 0, col);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm0 + i * 32 + 8 * (r / 4) + 4 * h + r % 4;
                if (row < M) {
                    float v = acc[i][j][r];
                    if (p.bias_mode == BIAS_COLUMN) v += col_bias;
                    else if (p.bias_mode == BIAS_ROW) v += bias[row];
                    C[col_offset + static_cast<long long>(row) * p.ldc] = activate(v, p.act, p.alpha);
                }
            }
    }
}

// C = act((float)(((0.0 + p0) + p1) + ... + p[S-1]) [+ bias]) with the FP64 sum in slice order,
// the bias (per column or per row) added in FP32 after the rounding, stored dense (row * ldc + col)
// or segmented like the GEMM's own epilogue.
__device__ __forceinline__ void finish_output(const GemmParams& p, float* C, long long i, double s) {
    const int row = static_cast<int>(i / p.N), col = static_cast<int>(i % p.N);
    float v = static_cast<float>(s);
    if (p.bias_mode == BIAS_COLUMN) v += p.bias[col];
    else if (p.bias_mode == BIAS_ROW) v += p.bias[row];
    C[output_offset(p, row, col)] = activate(v, p.act, p.alpha);
}

constexpr int REDUCE_AHEAD = 8;  // slices loaded before they are added

// One thread per output; the loads of REDUCE_AHEAD slices are issued before their additions, which
// still run one at a time in slice order.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ partial, float* __restrict__ C,
                                                           GemmParams p, int slices) {
    const long long i = blockIdx.x * 256LL + threadIdx.x, total = static_cast<long long>(p.M) * p.N;
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
    const long long q = blockIdx.x * 256LL + threadIdx.x, total = static_cast<long long>(p.M) * p.N;
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

using GemmFn = void (*)(GemmParams);
constexpr int VARIANTS = 16;  // 4 layouts (NN, NT, TN, TT) x float4 loads of A (yes/no) x of B

template <int T, bool TA, bool TB, bool VA, bool VB>
constexpr GemmFn kernel_of() {
    return gemm_mfma_kernel<TILES[T].bm, TILES[T].bn, TILES[T].bk, TILES[T].wm, TILES[T].wn, TA, TB, VA, VB>;
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
    }
};
static_assert(NUM_TILES == 8, "KernelTable lists every tile");

const KernelTable& kernel_table() {
    static const KernelTable table;
    return table;
}

int threads_of(const GemmTile& t) { return (t.bm / t.wm) * (t.bn / t.wn) * 64; }

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15) == 0; }

// Planner model of one workgroup tile: relative MFMA efficiency once latency is hidden, and how many
// workgroups fit on a CU at once (registers and LDS). Fitted to a sweep of every tile and split on
// MI355X over the ResNet18 batch-64 GEMM shapes and 4096^3.
struct TileCost {
    double efficiency;
    int per_cu;
};
constexpr TileCost COST[NUM_TILES] = {
    {1.063, 3}, {0.95, 3}, {0.85, 4}, {0.935, 6}, {0.60, 6}, {0.60, 6}, {1.02, 2}, {1.02, 2},
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
                                  ((t.bm / t.wm) * (t.bn / t.wn)) / 4.0;
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
GemmPlan gemm_auto_plan(int M, int N, int K, int batch) {
    GemmPlan best{0, 1, K};
    double best_cost = -1.0;
    for (int tile = 0; tile < NUM_TILES; ++tile) {
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
    return engine == 1 || (engine >= PLAN_BASE && engine < PLAN_BASE + NUM_TILES * MAX_SLICES);
}

int gemm_plan_from_engine(int engine, int M, int N, int K, GemmPlan* plan, int batch) {
    if (!gemm_engine_valid(engine)) return MFH_FAIL(ERR_ARG, "unknown GEMM engine or plan code");
    if (engine == 1) {
        *plan = gemm_auto_plan(M, N, K, batch);
        return OK;
    }
    const int code = engine - PLAN_BASE;
    const int tile = code / MAX_SLICES, requested = code % MAX_SLICES + 1;
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
    return p;
}

int launch_split_reduce(const float* partial, float* c, const GemmParams& p, int slices, hipStream_t stream) {
    const std::int64_t outputs = static_cast<std::int64_t>(p.M) * p.N;
    if (outputs % 4 == 0 && aligned16(partial)) {
        split_reduce_vec4_kernel<<<blocks_for(outputs / 4, 256), 256, 0, stream>>>(partial, c, p, slices);
        return MFH_CHECK_LAUNCH("split_reduce_vec4", stream);
    }
    split_reduce_kernel<<<blocks_for(outputs, 256), 256, 0, stream>>>(partial, c, p, slices);
    return MFH_CHECK_LAUNCH("split_reduce", stream);
}

}  // namespace

int split_reduce(const float* partial, float* c, int slices, int M, int N, int ldc, bool /*reference*/,
                 hipStream_t stream) {
    return launch_split_reduce(partial, c, epilogue_params(GemmEpilogue{}, M, N, ldc), slices, stream);
}

int gemm_launch(int engine, hipStream_t stream, const GemmOperands& o, const GemmEpilogue& e, float* workspace,
                std::int64_t workspace_floats) {
    const int M = o.M, N = o.N, K = o.K;
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
    } else {
        p.C = o.c;
        p.c_batch = o.c_batch;
        p.split = 0;
        p.k_chunk = K;
    }
    const int layout = (o.trans_a ? 2 : 0) + (o.trans_b ? 1 : 0);  // NN, NT, TN, TT
    const GemmFn fn = kernel_table().fn[plan.tile][layout * 4 + (vec_a ? 2 : 0) + (vec_b ? 1 : 0)];
    const dim3 grid(blocks_for(N, tile.bn), blocks_for(M, tile.bm), static_cast<unsigned>(planes));
    hipLaunchKernelGGL(fn, grid, dim3(threads_of(tile)), 0, stream, p);
    MFH_TRY(MFH_CHECK_LAUNCH("gemm_mfma", stream));
    if (!split) return OK;
    return launch_split_reduce(workspace, o.c, epilogue_params(e, M, N, o.ldc), plan.slices, stream);
}

}  // namespace mfh
