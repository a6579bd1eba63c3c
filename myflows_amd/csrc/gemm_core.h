// The MFMA main loop and epilogue shared by the dense GEMM engine (gemm.hip) and the implicit-GEMM
// convolution kernels (implicit.hip). Only the way a stage's operand tiles are read from global
// memory differs between them: a dense row copy, or a gather from an NCHW tensor.
//
// Work decomposition. A workgroup computes a BM x BN tile of C with (BM/WM) x (BN/WN) wave64s; a
// wave owns a WM x WN sub-tile made of (WM/32) x (WN/32) accumulators of v_mfma_f32_32x32x2_f32
// (16 floats per lane each). The K range of the workgroup is consumed in BK-deep stages that are
// double buffered in LDS: the global loads of stage t+1 are in flight while the waves run the
// MFMAs of stage t, with one barrier per stage.
//
// LDS layout. Each operand tile is kept in LDS in the orientation it has in global memory, so the
// global->LDS copy is a straight row copy with no transpose:
//   * "k-contiguous" operands (A when TA is false, B when TB is true) live as [rows][BK + 4];
//   * "mn-contiguous" operands (A when TA is true, B when TB is false) live as [BK][rows + 4].
// The +4 floats of padding keep 16-byte alignment and move successive rows to other banks.
//
// MFMA operand mapping. v_mfma_f32_32x32x2_f32 multiplies a 32x2 slice of A (lane l supplies
// A[l % 32][l / 32]) by a 2x32 slice of B (lane l supplies B[l / 32][l % 32]) and accumulates the
// 32x32 product; lane l holds output column l % 32, rows 8 * (r / 4) + 4 * (l / 32) + r % 4 in its
// register r. Which k a lane half (l / 32) feeds at each step is free as long as A and B agree, so
// half h consumes k = h * BK/2 + s for s = 0 .. BK/2 - 1 (or, with a pairing span below BK/2, the
// same within each sub-stage of MfmaShape::PAIR): a k-contiguous operand then reads four
// consecutive k of its row with one 16-byte LDS load. Every tile of one kernel family uses the same
// k mapping (the GEMM engine: pairs 8 apart in sub-stages of 16; the implicit products: stages of
// 32), so an unsplit product adds each output's K terms in the same order whatever the tile (of one
// K group: a K-grouped tile, gemm.hip, adds its groups' runs of stages afterwards).
#pragma once

#include <type_traits>

#include "common.h"

namespace mfh {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int GROUP_M = 8;  // tile rows per group of the tile order
constexpr int XCDS = 8;     // accelerator complex dies of an MI355X

// PAD_A / PAD_B: floats of padding after each LDS row. k-contiguous tiles need it (the float4
// reads of consecutive rows at one k would otherwise share banks); an mn-contiguous tile is read
// along its rows and can go without.
// PAIR: the k span between the two terms of one MFMA (lane half 1 reads k + PAIR where half 0
// reads k). With PAIR = BK / 2 (the default) half h consumes k = h * BK/2 + s of each stage; with a
// smaller PAIR the stage is consumed as BK / (2 * PAIR) sub-stages of depth 2 * PAIR in turn, each
// in that order, so a tile with deeper stages adds each output's terms in the same order, and to the
// same bits, as one whose stages are 2 * PAIR deep.
template <int BM_, int BN_, int BK_, int WM_, int WN_, bool TA_, bool TB_, int PAD_A = 4, int PAD_B = 4,
          int PAIR_ = BK_ / 2>
struct MfmaShape {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr bool TA = TA_, TB = TB_;
    static constexpr int WGN = BN / WN, WAVES = (BM / WM) * WGN, THREADS = WAVES * 64;
    static constexpr int TM = WM / 32, TN = WN / 32, HALF = BK / 2, PAIR = PAIR_;
    static_assert(PAIR % 4 == 0 && HALF % PAIR == 0, "a stage is whole sub-stages of groups of four k");
    static constexpr int LDA_S = TA ? BM + PAD_A : BK + PAD_A;  // LDS row lengths (floats)
    static constexpr int LDB_S = TB ? BK + PAD_B : BN + PAD_B;
    static constexpr int A_SIZE = TA ? BK * LDA_S : BM * LDA_S;
    static constexpr int B_SIZE = TB ? BN * LDB_S : BK * LDB_S;
    static constexpr int STAGE = A_SIZE + B_SIZE;
    static_assert(BK % 8 == 0, "each lane half consumes groups of four k");
};

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

// Buffer loads (the raw buffer instructions of CDNA): a 128-bit resource in SGPRs holds the base
// address and the byte extent of one tensor; each load adds a per-lane byte offset (VGPR) and a
// wave-uniform one (SGPR). A lane whose offset lies past the extent reads zero without touching
// memory, so a gather marks its out-of-image lanes with BUFFER_OOB instead of branching around the
// load, and the address arithmetic that is the same for the whole wave stays in scalar registers.
// The extent must fit in 31 bits (BUFFER_LIMIT_FLOATS); BUFFER_OOB then lies beyond every extent,
// also after a wave-uniform offset inside the extent is added to it.
constexpr unsigned BUFFER_OOB = 0x80000000u;
constexpr int BUFFER_CONFIG = 0x00020000;  // resource word 3 for gfx9-family raw buffers (stride 0)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const float* base, long long floats) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0),
                                             static_cast<int>(floats * 4), BUFFER_CONFIG);
}

__device__ __forceinline__ float buffer_load(__amdgpu_buffer_rsrc_t r, unsigned lane_bytes, int wave_bytes) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, lane_bytes, wave_bytes, 0));
}

__device__ __forceinline__ float4 buffer_load4(__amdgpu_buffer_rsrc_t r, unsigned lane_bytes, int wave_bytes) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, lane_bytes, wave_bytes, 0));
}

// A ROWS x COLS tile of a row-major matrix (rows of length ld, `rows` of them) whose COLS columns
// [col0, col0 + COLS) lie inside every row: float4 buffer loads, the column offset wave-uniform;
// rows past the end read zero. COLS a multiple of 4, ld a multiple of 4, base 16-byte aligned.
template <int ROWS, int COLS, int THREADS>
struct BufferRowTile {
    static constexpr int VCOLS = COLS / 4, ELEMS = ROWS * VCOLS;
    static constexpr int PER_THREAD = (ELEMS + THREADS - 1) / THREADS;
    __amdgpu_buffer_rsrc_t rsrc;
    unsigned lane_bytes[PER_THREAD];
    float4 v[PER_THREAD];

    __device__ __forceinline__ void init(const float* base, int ld, int rows, int row0, int tid) {
        rsrc = buffer_of(base, static_cast<long long>(rows) * ld);
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) {
            const int f = tid + i * THREADS;
            const int row = row0 + f / VCOLS;
            lane_bytes[i] = f < ELEMS && row < rows ? static_cast<unsigned>(row * ld + f % VCOLS * 4) * 4u : BUFFER_OOB;
        }
    }

    __device__ __forceinline__ void load(int col0) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) v[i] = buffer_load4(rsrc, lane_bytes[i], col0 * 4);
    }

    template <int LD>
    __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) {
            const int f = tid + i * THREADS;
            if (ELEMS % THREADS == 0 || f < ELEMS) *reinterpret_cast<float4*>(lds + f / VCOLS * LD + f % VCOLS * 4) = v[i];
        }
    }
};

__device__ __forceinline__ float activate(float v, int act, float alpha) {
    if (act == ACT_RELU) return v < 0.0f ? 0.0f : v;  // NaN stays NaN
    if (act == ACT_LEAKY_RELU) return v > 0.0f ? v : alpha * v;
    return v;
}

// Where output (row, col) lives: dense row * ldc + col, or segmented (column j is element j % segment
// of segment j / segment, segments segment_stride apart, the element spread over a lattice when
// p.lattice_w is set), after mapping a chunked-order feature column back to its natural index when
// p.taps is set.
__device__ __forceinline__ long long output_offset(const GemmParams& p, int row, int col) {
    if (p.taps) {  // chunked feature order -> natural order c * taps + tap
        int tap;
        const int chunk = p.taps_div.divmod(col / CHANNEL_CHUNK, tap);
        col = (chunk * CHANNEL_CHUNK + col % CHANNEL_CHUNK) * p.taps + tap;
    }
    if (p.segment) {
        int within;
        const int segment = p.segment_div.divmod(col, within);
        if (p.lattice_w) {
            int j;
            const int i = p.lattice_div.divmod(within, j);
            within = i * p.lattice_row + j * p.lattice_col + p.lattice_offset;
        }
        return segment * p.segment_stride + static_cast<long long>(row) * p.ldc + within;
    }
    return static_cast<long long>(row) * p.ldc + col;
}

// The zeros of output (row, col)'s lattice cell besides the output itself (GemmParams::cell_h).
__device__ __forceinline__ void zero_cell(const GemmParams& p, float* __restrict__ C, int row, int col) {
    int within, j;
    const int segment = p.segment_div.divmod(col, within);
    const int i = p.lattice_div.divmod(within, j);
    float* base = C + segment * p.segment_stride + static_cast<long long>(row) * p.ldc;
    for (int a = 0; a < p.cell_h; ++a) {
        const int h = p.cell_h * i + a;
        if (h >= p.plane_h) break;
        for (int b = 0; b < p.cell_w; ++b) {
            const int w = p.cell_w * j + b;
            if (w >= p.plane_w) break;
            if (a | b) base[h * p.plane_w + w] = 0.0f;
        }
    }
}

// One output: stored (or added, with p.accumulate) where output_offset puts it, and its lattice
// cell's other positions zeroed when p.cell_h is set.
__device__ __forceinline__ void write_output(const GemmParams& p, float* __restrict__ C, int row, int col, float v) {
    float* out = C + output_offset(p, row, col);
    *out = p.accumulate ? *out + v : v;
    if (p.cell_h) zero_cell(p, C, row, col);
}

// (tile row, tile column, z) of this workgroup. Workgroups are handed to the 8 XCDs round-robin by
// their linear id, and each XCD has its own L2: the renumbering gives XCD x one contiguous run of
// tiles, walked in groups of GROUP_M tile rows (column by column inside a group), so the tiles an
// XCD runs at the same time share A row panels and B column panels in its L2.
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

template <class S>
__device__ __forceinline__ void zero_acc(v16f (&acc)[S::TM][S::TN]) {
#pragma unroll
    for (int i = 0; i < S::TM; ++i)
#pragma unroll
        for (int j = 0; j < S::TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
}

// One stage of MFMAs on the LDS tiles As / Bs (see the operand mapping above).
// KK0 / KK1 select a part of the stage (groups of four k per lane half), for a loop that puts
// other work between the parts. RESTART: the part's first MFMA takes a zero accumulator input, so
// the accumulators start over with this stage (their earlier contents are discarded).
template <class S, int KK0 = 0, int KK1 = S::HALF, bool RESTART = false>
__device__ __forceinline__ void mfma_stage(const float* As, const float* Bs, v16f (&acc)[S::TM][S::TN], int wm0,
                                           int wn0, int lane) {
    constexpr int PAIR = S::PAIR, LDA_S = S::LDA_S, LDB_S = S::LDB_S;
    const int lm = lane % 32, h = lane / 32;
#pragma unroll
    for (int kk = KK0; kk < KK1; kk += 4) {
        const int k = kk / PAIR * 2 * PAIR + h * PAIR + kk % PAIR;
        float4 a[S::TM], b[S::TN];
#pragma unroll
        for (int i = 0; i < S::TM; ++i) {
            const int m = wm0 + i * 32 + lm;
            if constexpr (S::TA)
                a[i] = make_float4(As[k * LDA_S + m], As[(k + 1) * LDA_S + m], As[(k + 2) * LDA_S + m],
                                   As[(k + 3) * LDA_S + m]);
            else a[i] = *reinterpret_cast<const float4*>(As + m * LDA_S + k);
        }
#pragma unroll
        for (int j = 0; j < S::TN; ++j) {
            const int n = wn0 + j * 32 + lm;
            if constexpr (S::TB) b[j] = *reinterpret_cast<const float4*>(Bs + n * LDB_S + k);
            else
                b[j] = make_float4(Bs[k * LDB_S + n], Bs[(k + 1) * LDB_S + n], Bs[(k + 2) * LDB_S + n],
                                   Bs[(k + 3) * LDB_S + n]);
        }
#pragma unroll
        for (int i = 0; i < S::TM; ++i)
#pragma unroll
            for (int j = 0; j < S::TN; ++j) {
                if (RESTART && kk == KK0)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].x, b[j].x, v16f{}, 0, 0, 0);
                else
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
            }
    }
}

// Instruction order inside a stage, chosen per kernel by measurement on MI355X (the arithmetic and
// its order are the same for all of them):
//   STAGE_PLAIN     MFMAs of the stage, then the LDS store of the next stage, then the barrier;
//   STAGE_PRIORITY  the same, with the wave's issue priority raised (s_setprio 1) from the start of
//                   its MFMAs to the barrier, so that waves in their MFMA phase issue first while
//                   the others store and wait: 4 % on the dense 256x128 GEMM;
//   STAGE_MID_STORE the LDS store of the next stage between the first and the second half of the
//                   stage's MFMAs: 3-5 % on the dW products, whose stores carry gathered operands;
//   STAGE_EARLY_STORE the store after the first quarter of the stage's MFMAs (stages of at least
//                   32 k): 3 % on the 256x256 GEMM tile (one workgroup per CU, where a raised
//                   priority only delays the other waves' stores) and 1 % on the batch-64 training
//                   step through the forward / dX products, whose reads run two stages ahead.
enum StageOrder : int { STAGE_PLAIN = 0, STAGE_PRIORITY = 1, STAGE_MID_STORE = 2, STAGE_EARLY_STORE = 3 };

// What a K loop does with the accumulators after each stage's MFMAs: nothing (the FP32 chain runs
// on over the whole K range), or StageSums below (restarts = whether each stage starts its
// accumulators from zero).
struct KeepChain {
    static constexpr bool restarts = false;
    template <class Acc>
    __device__ __forceinline__ void operator()(Acc&) const {}
};

// Stage sums: each stage's BK terms are summed on the matrix cores into accumulators that start
// from zero, and the stage sums are then added to totals of type T, so an output's rounding chain
// on the matrix cores is one stage long instead of the whole K range: a two-level sum, whose error
// grows like sqrt(BK * K + K^2 / BK) unit roundoffs instead of K for one chain (T = float), or like
// sqrt(BK * K) (T = double, at twice the registers). rounded() gives the totals as float. The drain
// of stage t runs at the start of stage t + 1, after the barrier, when the stage's MFMAs are done.
template <class S, class T = double>
struct StageSums {
    static constexpr bool restarts = true;
    T total[S::TM][S::TN][16];
    __device__ __forceinline__ StageSums() {
#pragma unroll
        for (int i = 0; i < S::TM; ++i)
#pragma unroll
            for (int j = 0; j < S::TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) total[i][j][r] = T(0);
    }
    __device__ __forceinline__ void operator()(v16f (&acc)[S::TM][S::TN]) {
#pragma unroll
        for (int i = 0; i < S::TM; ++i)
#pragma unroll
            for (int j = 0; j < S::TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) total[i][j][r] += static_cast<T>(acc[i][j][r]);
    }
    __device__ __forceinline__ void rounded(v16f (&acc)[S::TM][S::TN]) const {
#pragma unroll
        for (int i = 0; i < S::TM; ++i)
#pragma unroll
            for (int j = 0; j < S::TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = static_cast<float>(total[i][j][r]);
    }
};

// The K loop over [k_begin, k_end) in BK stages. fetch(kt) issues the global reads of the stage
// starting at kt; store(a_lds, b_lds) writes the fetched registers into one LDS stage buffer;
// drain(acc) runs after each stage's MFMAs (KeepChain or StageSums).
template <class S, int ORDER = STAGE_PLAIN, class Fetch, class Store, class Drain = KeepChain>
__device__ __forceinline__ void mfma_k_loop(float* smem, int k_begin, int k_end, Fetch&& fetch, Store&& store,
                                            v16f (&acc)[S::TM][S::TN], int wm0, int wn0, int lane,
                                            Drain&& drain = Drain{}) {
    constexpr int BK = S::BK;
    const int stages = k_end > k_begin ? (k_end - k_begin + BK - 1) / BK : 0;
    if (stages > 0) {
        fetch(k_begin);
        store(smem, smem + S::A_SIZE);
    }
    __syncthreads();
    for (int t = 0; t < stages; ++t) {
        const bool more = t + 1 < stages;
        if (more) fetch(k_begin + (t + 1) * BK);
        // The previous stage's sums: its MFMAs have completed while the wave waited at the barrier.
        if (t > 0) drain(acc);
        const float* As = smem + (t & 1) * S::STAGE;
        float* next = smem + ((t + 1) & 1) * S::STAGE;
        constexpr bool RESTART = std::decay_t<Drain>::restarts;
        if constexpr ((ORDER == STAGE_MID_STORE && S::HALF >= 8) || (ORDER == STAGE_EARLY_STORE && S::HALF >= 16)) {
            constexpr int MID = ORDER == STAGE_EARLY_STORE ? S::HALF / 16 * 4 : S::HALF / 8 * 4;
            mfma_stage<S, 0, MID, RESTART>(As, As + S::A_SIZE, acc, wm0, wn0, lane);
            if (more) store(next, next + S::A_SIZE);
            mfma_stage<S, MID, S::HALF>(As, As + S::A_SIZE, acc, wm0, wn0, lane);
        } else {
            if constexpr (ORDER == STAGE_PRIORITY) __builtin_amdgcn_s_setprio(1);
            mfma_stage<S, 0, S::HALF, RESTART>(As, As + S::A_SIZE, acc, wm0, wn0, lane);
            if (more) store(next, next + S::A_SIZE);
            if constexpr (ORDER == STAGE_PRIORITY) __builtin_amdgcn_s_setprio(0);
        }
        __syncthreads();
    }
    if (stages > 0) drain(acc);
}

// The K loop with the global reads two stages ahead: the reads of stage t + 2 are issued when stage
// t starts, into one of two register slots, so a stage's reads have two stages of MFMAs to arrive
// before they are stored to LDS (at the end of stage t + 1) instead of one. fetch(slot, kt) and
// store(slot, a_lds, b_lds) take the slot as std::integral_constant<int, 0 or 1>: stage t uses slot
// t % 2 and LDS buffer t % 2. The MFMAs, their operands and their order are mfma_k_loop's (with
// ORDER STAGE_PLAIN, STAGE_MID_STORE or STAGE_EARLY_STORE), so the results are its bits. fetch is issued for every stage, also for the two past
// the end (kt >= k_end), and store for every stage, also for the one past the end (into the LDS
// buffer that no MFMA reads any more: every wave has passed the barrier after its last read), so
// that the compiler sees the same loads in flight on every path and waits for exactly one stage's
// (a conditional store makes it wait for the other slot's loads at the top of a stage): a loader
// must read nothing (or stay in bounds) past the end, as the buffer loaders do, whose out-of-range
// lanes read zero, and a store's side effects must not mind the zeros.
template <class S, int ORDER = STAGE_PLAIN, class Fetch, class Store, class Drain = KeepChain>
__device__ __forceinline__ void mfma_k_loop_ahead(float* smem, int k_begin, int k_end, Fetch&& fetch, Store&& store,
                                                  v16f (&acc)[S::TM][S::TN], int wm0, int wn0, int lane,
                                                  Drain&& drain = Drain{}) {
    constexpr int BK = S::BK;
    using Slot0 = std::integral_constant<int, 0>;
    using Slot1 = std::integral_constant<int, 1>;
    const int stages = k_end > k_begin ? (k_end - k_begin + BK - 1) / BK : 0;
    if (stages > 0) {
        fetch(Slot0{}, k_begin);
        fetch(Slot1{}, k_begin + BK);
        store(Slot0{}, smem, smem + S::A_SIZE);
    }
    __syncthreads();
    constexpr bool RESTART = std::decay_t<Drain>::restarts;
    // Stage t of slot T: fetch stage t + 2 into slot T, the MFMAs of LDS buffer T, then stage t + 1
    // (slot 1 - T) into LDS buffer 1 - T.
    auto stage = [&](auto slot, int t) {
        constexpr int T = decltype(slot)::value;
        using Other = std::integral_constant<int, 1 - T>;
        fetch(slot, k_begin + (t + 2) * BK);
        if (t > 0) drain(acc);
        const float* As = smem + T * S::STAGE;
        float* next = smem + (1 - T) * S::STAGE;
        if constexpr ((ORDER == STAGE_MID_STORE && S::HALF >= 8) || (ORDER == STAGE_EARLY_STORE && S::HALF >= 16)) {
            constexpr int MID = ORDER == STAGE_EARLY_STORE ? S::HALF / 16 * 4 : S::HALF / 8 * 4;
            mfma_stage<S, 0, MID, RESTART>(As, As + S::A_SIZE, acc, wm0, wn0, lane);
            store(Other{}, next, next + S::A_SIZE);
            mfma_stage<S, MID, S::HALF>(As, As + S::A_SIZE, acc, wm0, wn0, lane);
        } else {
            mfma_stage<S, 0, S::HALF, RESTART>(As, As + S::A_SIZE, acc, wm0, wn0, lane);
            store(Other{}, next, next + S::A_SIZE);
        }
        __syncthreads();
    };
    // Pairs of stages, then an odd last one: a loop body that could skip its second stage would
    // leave the compiler a path back to the first with that stage's loads still in flight, and it
    // would then wait for them at the top of every pair.
    int t = 0;
    for (; t + 1 < stages; t += 2) {
        stage(Slot0{}, t);
        stage(Slot1{}, t + 1);
    }
    if (t < stages) stage(Slot0{}, t);
    if (stages > 0) drain(acc);
}

// Epilogue: bias (per output column or per output row), the activation, then the store of the
// wave's accumulators into C (dense or segmented, see output_offset), added to what C holds when
// p.accumulate.
template <class S>
__device__ __forceinline__ void store_acc(const GemmParams& p, float* __restrict__ C, const v16f (&acc)[S::TM][S::TN],
                                          int m0, int n0, int wm0, int wn0, int lane) {
    const int lm = lane % 32, h = lane / 32;
    const float* __restrict__ bias = p.bias;
#pragma unroll
    for (int j = 0; j < S::TN; ++j) {
        const int col = n0 + wn0 + j * 32 + lm;
        if (col >= p.N) continue;
        const float col_bias = p.bias_mode == BIAS_COLUMN ? bias[col] : 0.f;
        const long long col_offset = output_offset(p, 0, col);
#pragma unroll
        for (int i = 0; i < S::TM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm0 + i * 32 + 8 * (r / 4) + 4 * h + r % 4;
                if (row < p.M) {
                    float v = acc[i][j][r];
                    if (p.bias_mode == BIAS_COLUMN) v += col_bias;
                    else if (p.bias_mode == BIAS_ROW) v += bias[row];
                    const long long offset = col_offset + static_cast<long long>(row) * p.ldc;
                    if (p.residual) v = v + p.residual[offset];
                    float* out = C + offset;
                    v = activate(v, p.act, p.alpha);
                    *out = p.accumulate ? *out + v : v;
                    if (p.cell_h) zero_cell(p, C, row, col);
                }
            }
    }
}

}  // namespace mfh
