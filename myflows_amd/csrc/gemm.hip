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
// consecutive k of its row with one 16-byte LDS load.
//
// The third grid dimension has two uses:
//   * split-K (GemmParams::split = 1): z selects the K slice [z * k_chunk, min(K, (z+1) * k_chunk))
//     and writes its partial product to C + z * c_batch; split_reduce then sums the slices in a fixed
//     order in FP64;
//   * batches (split = 0): z is an independent problem at A + z * a_batch, B + z * b_batch,
//     C + z * c_batch (one per image for the convolution's per-image GEMMs).
// Every output element is produced by one wave in one fixed order, so results are bitwise
// reproducible run to run.
#include "common.h"

namespace mfh {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

// Tile catalogue: block tile BM x BN, stage depth BK, wave tile WM x WN (multiples of 32).
constexpr GemmTile TILES[] = {
    {128, 128, 16, 64, 64},  // 0: general
    {256, 64, 16, 64, 64},   // 1: tall outputs, N <= 64 (convolution forward rows)
    {64, 128, 16, 32, 64},   // 2: short outputs, M <= 64 (weight gradients)
    {64, 64, 16, 32, 32},    // 3: small outputs
    {128, 32, 16, 32, 32},   // 4: N <= 32
    {32, 128, 16, 32, 32},   // 5: M <= 32
    {256, 128, 16, 64, 64},  // 6: large square-ish outputs, 8 waves
    {128, 256, 16, 64, 64},  // 7: large square-ish outputs, 8 waves
};
constexpr int NUM_TILES = sizeof(TILES) / sizeof(TILES[0]);
constexpr int PLAN_BASE = 16;     // engine codes >= PLAN_BASE name a tile and a slice count
constexpr int MAX_SLICES = 128;   // slices per explicit plan code
constexpr int MIN_CHUNK = 128;    // smallest K slice the automatic planner makes

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

template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, bool VEC>
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

    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int lm = lane % 32, h = lane / 32;
    const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int z = blockIdx.z;
    const float* __restrict__ A = p.A + (p.split ? 0 : z * p.a_batch);
    const float* __restrict__ B = p.B + (p.split ? 0 : z * p.b_batch);
    float* __restrict__ C = p.C + z * p.c_batch;
    const int k_begin = p.split ? z * p.k_chunk : 0;
    const int k_end = p.split ? min(p.K, k_begin + p.k_chunk) : p.K;
    const int M = p.M, N = p.N;

    // A tile: rows = m (k-contiguous) or k (mn-contiguous); likewise B.
    TileLoader<TA ? BK : BM, TA ? BM : BK, THREADS, VEC> la;
    TileLoader<TB ? BN : BK, TB ? BK : BN, THREADS, VEC> lb;
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

    // Epilogue: bias (per output column or per output row), then the activation, then the store.
    const float* __restrict__ bias = p.bias;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn0 + j * 32 + lm;
        const float col_bias = p.bias_mode == BIAS_COLUMN && col < N ? bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm0 + i * 32 + 8 * (r / 4) + 4 * h + r % 4;
                if (row < M && col < N) {
                    float v = acc[i][j][r];
                    if (p.bias_mode == BIAS_COLUMN) v += col_bias;
                    else if (p.bias_mode == BIAS_ROW) v += bias[row];
                    C[static_cast<long long>(row) * p.ldc + col] = activate(v, p.act, p.alpha);
                }
            }
    }
}

// C = act((float)(((0.0 + p0) + p1) + ... + p[S-1]) [+ bias]) with the FP64 sum in slice order,
// the bias (per column or per row) added in FP32 after the rounding.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ partial, float* __restrict__ C,
                                                           const float* __restrict__ bias, int bias_mode, int act,
                                                           float alpha, int slices, int M, int N, int ldc) {
    const long long i = blockIdx.x * 256LL + threadIdx.x, total = static_cast<long long>(M) * N;
    if (i >= total) return;
    double s = 0.0;
    for (int z = 0; z < slices; ++z) s += static_cast<double>(partial[z * total + i]);
    const long long row = i / N, col = i % N;
    float v = static_cast<float>(s);
    if (bias_mode == BIAS_COLUMN) v += bias[col];
    else if (bias_mode == BIAS_ROW) v += bias[row];
    C[row * ldc + col] = activate(v, act, alpha);
}

using GemmFn = void (*)(GemmParams);
constexpr int VARIANTS = 8;  // 4 layouts (NN, NT, TN, TT) x scalar / float4 loads

template <int T, bool TA, bool TB, bool VEC>
constexpr GemmFn kernel_of() {
    return gemm_mfma_kernel<TILES[T].bm, TILES[T].bn, TILES[T].bk, TILES[T].wm, TILES[T].wn, TA, TB, VEC>;
}

template <int T>
constexpr void fill_row(GemmFn (&row)[VARIANTS]) {
    row[0] = kernel_of<T, false, false, false>();
    row[1] = kernel_of<T, false, false, true>();
    row[2] = kernel_of<T, false, true, false>();
    row[3] = kernel_of<T, false, true, true>();
    row[4] = kernel_of<T, true, false, false>();
    row[5] = kernel_of<T, true, false, true>();
    row[6] = kernel_of<T, true, true, false>();
    row[7] = kernel_of<T, true, true, true>();
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

int tile_for_shape(int M, int N) {
    if (N <= 32) return 4;
    if (M <= 32) return 5;
    if (N <= 64) return M <= 64 ? 3 : 1;
    if (M <= 64) return 2;
    return 0;
}

}  // namespace

int gemm_tile_count() { return NUM_TILES; }
const GemmTile& gemm_tile(int index) { return TILES[index]; }

// Tile by output shape; split K when the output covers fewer than two workgroups per CU and K is
// long relative to the output (K >= M + N): the weight-gradient GEMMs, whose K is the pixel count.
GemmPlan gemm_auto_plan(int M, int N, int K) {
    const int tile = tile_for_shape(M, N);
    GemmPlan plan{tile, 1, K};
    const std::int64_t tiles = static_cast<std::int64_t>(blocks_for(M, TILES[tile].bm)) * blocks_for(N, TILES[tile].bn);
    const std::int64_t target = 2LL * device_cu_count();
    if (tiles >= target || K < static_cast<std::int64_t>(M) + N) return plan;
    const std::int64_t split =
        std::min<std::int64_t>({(target + tiles - 1) / tiles, K / MIN_CHUNK, static_cast<std::int64_t>(MAX_SLICES)});
    if (split < 2) return plan;
    const int bk = TILES[tile].bk;
    plan.k_chunk = static_cast<int>(((K + split - 1) / split + bk - 1) / bk * bk);
    plan.slices = (K + plan.k_chunk - 1) / plan.k_chunk;
    return plan;
}

bool gemm_engine_valid(int engine) {
    return engine == 1 || (engine >= PLAN_BASE && engine < PLAN_BASE + NUM_TILES * MAX_SLICES);
}

int gemm_plan_from_engine(int engine, int M, int N, int K, GemmPlan* plan) {
    if (!gemm_engine_valid(engine)) return MFH_FAIL(ERR_ARG, "unknown GEMM engine or plan code");
    if (engine == 1) {
        *plan = gemm_auto_plan(M, N, K);
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

int split_reduce_epilogue(const float* partial, float* c, const GemmEpilogue& e, int slices, int M, int N, int ldc,
                          hipStream_t stream) {
    const std::int64_t outputs = static_cast<std::int64_t>(M) * N;
    split_reduce_kernel<<<blocks_for(outputs, 256), 256, 0, stream>>>(partial, c, e.bias, e.bias_mode, e.act, e.alpha,
                                                                        slices, M, N, ldc);
    return MFH_CHECK_LAUNCH("split_reduce", stream);
}

int split_reduce(const float* partial, float* c, int slices, int M, int N, int ldc, bool /*reference*/,
                 hipStream_t stream) {
    return split_reduce_epilogue(partial, c, GemmEpilogue{}, slices, M, N, ldc, stream);
}

int gemm_launch(int engine, hipStream_t stream, const GemmOperands& o, const GemmEpilogue& e, float* workspace,
                std::int64_t workspace_floats) {
    const int M = o.M, N = o.N, K = o.K;
    GemmPlan plan;
    MFH_TRY(gemm_plan_from_engine(engine, M, N, K, &plan));
    if (o.batch > 1 || (plan.slices > 1 && (!workspace || workspace_floats < gemm_workspace_floats(plan, M, N))))
        plan = GemmPlan{plan.tile, 1, K};
    const bool split = plan.slices > 1;
    // float4 loads need the contiguous extent of each operand, its leading dimension, its batch
    // stride and its base pointer to be multiples of 4 floats / 16 bytes; K slices are multiples of BK.
    const bool vec = (o.trans_a ? M : K) % 4 == 0 && (o.trans_b ? K : N) % 4 == 0 && o.lda % 4 == 0 &&
                     o.ldb % 4 == 0 && o.a_batch % 4 == 0 && o.b_batch % 4 == 0 && aligned16(o.a) && aligned16(o.b);
    const GemmTile& tile = TILES[plan.tile];
    if (blocks_for(M, tile.bm) > GRID_YZ_LIMIT) return MFH_FAIL(ERR_ARG, "GEMM rows exceed the grid limit");
    if (static_cast<unsigned>(o.batch) > GRID_YZ_LIMIT) return MFH_FAIL(ERR_ARG, "GEMM batch exceeds the grid limit");
    GemmParams p{};
    p.A = o.a;
    p.B = o.b;
    p.M = M;
    p.N = N;
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
    } else {
        p.C = o.c;
        p.ldc = o.ldc;
        p.c_batch = o.c_batch;
        p.split = 0;
        p.k_chunk = K;
        p.bias = e.bias;
        p.bias_mode = e.bias_mode;
        p.act = e.act;
        p.alpha = e.alpha;
    }
    const int layout = (o.trans_a ? 2 : 0) + (o.trans_b ? 1 : 0);  // NN, NT, TN, TT
    const GemmFn fn = kernel_table().fn[plan.tile][layout * 2 + (vec ? 1 : 0)];
    const dim3 grid(blocks_for(N, tile.bn), blocks_for(M, tile.bm), split ? plan.slices : o.batch);
    hipLaunchKernelGGL(fn, grid, dim3(threads_of(tile)), 0, stream, p);
    MFH_TRY(MFH_CHECK_LAUNCH("gemm_mfma", stream));
    if (!split) return OK;
    return split_reduce_epilogue(workspace, o.c, e, plan.slices, M, N, o.ldc, stream);
}

}  // namespace mfh
