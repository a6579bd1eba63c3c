/*
 * libmfhip: the MI355X (gfx950) native library behind MyFlows' convolution / GEMM / max-pool hot
 * path and the batch-norm, ReLU and Adam kernels of the training step around it. It replaces the
 * NVRTC + cuBLAS scheduler of the reference (ops/cuda_native/native_cublas.cpp) and the CuPy
 * kernels of ops/fused.py behind the same calling conventions:
 *
 *   - every device buffer is a uint64_t device address owned by the caller (PyTorch here, CuPy in
 *     the reference); the library never allocates device memory (its one device array, the fixed
 *     scratch of mfh_gemm_noalloc, is part of the loaded code object);
 *   - a null optional pointer means "not requested";
 *   - dimensions are int, the stream is a uint64_t hipStream_t handle (0 = null stream);
 *   - launches are asynchronous on that stream; nothing synchronises unless debug sync is on
 *     (mfh_set_debug_sync(1) or MFHIP_SYNC=1);
 *   - every entry point returns a status: 0 OK, 1 initialisation failed, 2 invalid argument,
 *     3 HIP runtime error, 5 called on another device than mfh_init's (4 is unused; it was the
 *     cuBLAS status of the reference). The detail is this thread's mfh_last_error(), of the form
 *     "<file>:<line>: <reason>".
 *
 * Kernels index buffers with int32 offsets; entry points reject problems whose buffers exceed
 * 2^31 - 1 elements.
 *
 * GEMM engine codes (engine arguments), with the reference's arithmetic: 1 = the FP32 MFMA engine
 * with its automatic tile and split-K plan; 16 + n * 32 + (slices - 1) = the reference's named tile n
 * (0 128x128, 1 128x64, 2 256x32, 3 64x128, 4 32x256; 1..32 K slices), run on this library's tile of
 * the same role (128x128, 256x64, 128x32, 64x128, 32x128); 1024 + tile * 128 + (slices - 1) = tile
 * `tile` of this library's catalogue (mfh_gemm_tile_info), 1..128 K slices. Extended codes index the
 * catalogue of the library that decodes them, so they carry over between builds by tile name only.
 * The reference's engine 0 (cuBLAS) does not exist here. (The implicit convolution entry points have
 * their own plan codes: 16 + tile * 128 + (slices - 1) over the 12 implicit tiles.)
 */
#ifndef MFHIP_H
#define MFHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MFH_API __attribute__((visibility("default")))

/* ---- library -------------------------------------------------------------------------------- */

/* One-time initialisation on the current HIP device: checks that the device is gfx950, that the
 * embedded code objects load, reads the CU count and the MFHIP_SYNC flag.
 * Replaces mf_init(cublas_path, nvrtc_path, cache_dir), ops/cuda_native/native_cublas.cpp:1425-1427
 * (no library paths and no kernel cache: code objects are compiled ahead of time). */
MFH_API int mfh_init(void);

/* Replaces mf_last_error, native_cublas.cpp:1413-1415. */
MFH_API const char* mfh_last_error(void);

/* JSON build/device facts: device_arch, device_name, cu_count, binary, load_ms.
 * Replaces mf_info, native_cublas.cpp:1417-1419. */
MFH_API const char* mfh_info(void);

/* Synchronise the stream after every launch so asynchronous faults name their kernel.
 * Replaces mf_set_debug_sync, native_cublas.cpp:1421-1423. */
MFH_API void mfh_set_debug_sync(int enabled);

/* Stream order: nothing issued on `waiting` after this call starts before all the work issued so
 * far on `signalling` has finished (an event recorded on one, waited for by the other; the host
 * does not block). Both are streams of the current device; the same stream twice is a no-op. The
 * event carries no system-scope fence: it orders the device's streams (the memory the signalling
 * stream's kernels wrote is visible to the waiting stream's), not the host, which synchronises
 * through its own stream or device synchronisation.
 * No counterpart in the reference, whose operators run on one stream: for callers that issue work
 * on a second stream, such as the dW products of a backward pass beside its dX products. */
MFH_API int mfh_stream_wait(uint64_t waiting, uint64_t signalling);

/* ---- recorded programs ---------------------------------------------------------------------- */

/* Start recording, on the calling thread, every kernel launch and stream ordering the library
 * issues from now on (they still run as usual) into a program, until mfh_program_end. Status 2 when
 * this thread already records one.
 * No counterpart in the reference: for a caller that issues the same sequence of library calls
 * (a training step) again and again and whose host time would otherwise bound it. */
MFH_API int mfh_program_begin(void);

/* Stop recording: *program receives a handle to the recorded steps and *launches (when not null)
 * the number of kernel launches among them. The handle stays valid until mfh_program_free. */
MFH_API int mfh_program_end(uint64_t* program, int64_t* launches);

/* Issue the recorded steps again, in their order and on their streams: the same kernels with the
 * same arguments and buffers, without the host work that chose them. The caller keeps every buffer
 * and stream of the recording alive, and refreshes inputs in place; work that other libraries did
 * during the recording is not part of the program. Status 3 names the step whose launch failed. */
MFH_API int mfh_program_run(uint64_t program);

/* Release a program handle from mfh_program_end. */
MFH_API void mfh_program_free(uint64_t program);

/* p[0 .. count) = value (float32), on `stream`. No counterpart in the reference (whose graph seeds
 * its backward with xp.ones): the seed of a backward pass as a library launch, so that a recorded
 * program makes it too. */
MFH_API int mfh_fill(uint64_t p, int64_t count, float value, uint64_t stream);

/* ---- convolution ---------------------------------------------------------------------------- */

/* cols (N*OH*OW, CI*KH*KW) = im2col(x), zero outside the padded input.
 * Replaces mf_conv_im2col, native_cublas.cpp:1430-1438. */
MFH_API int mfh_conv_im2col(uint64_t x, uint64_t cols, int N, int CI, int H, int W, int CO, int KH, int KW, int OH,
                            int OW, int SH, int SW, int PH, int PW, uint64_t stream);

/* dx (N, CI, H, W) = col2im of a feature-major column gradient: the sum, over every window position
 * that reads an input position, of that position's column-gradient entry, in a fixed order (so the
 * result is deterministic). grad_cols is [n][CI*KH*KW][OH*OW] when per_image, else
 * [CI*KH*KW][N*OH*OW]; with accumulate, dx += the sums.
 * No counterpart of its own in the reference, whose col2im (native_cublas.cpp:247-271, over the
 * pixel-major grad_cols) runs inside mf_conv_backward_plans: for callers that form the column
 * gradient themselves, and to time the col2im pass alone. */
MFH_API int mfh_conv_col2im(uint64_t grad_cols, uint64_t dx, int N, int CI, int H, int W, int CO, int KH, int KW,
                            int OH, int OW, int SH, int SW, int PH, int PW, int per_image, int accumulate,
                            uint64_t stream);

/* y (N,CO,OH,OW) = act(conv(x, weight) + bias). cols receives im2col(x) (kept by the caller for
 * dW). With rows == 0 one GEMM W cols^T over all images writes y straight into NCHW, bias and
 * activation in its epilogue (workspace: the mfh_gemm_workspace(CO, N*OH*OW, CI*KH*KW) floats that
 * let it split K, or 0); with rows (N*OH*OW x CO floats) given, rows = cols W^T is formed first
 * (workspace: mfh_gemm_workspace(N*OH*OW, CO, CI*KH*KW)) and an epilogue kernel transposes it.
 * activation: 0 none, 1 ReLU, 2 LeakyReLU(alpha > 0). bias may be 0.
 * Replaces mf_conv_forward, native_cublas.cpp:1441-1461. */
MFH_API int mfh_conv_forward(uint64_t x, uint64_t weight, uint64_t bias, uint64_t cols, uint64_t rows, uint64_t y,
                             int N, int CI, int H, int W, int CO, int KH, int KW, int OH, int OW, int SH, int SW,
                             int PH, int PW, int activation, float alpha, int engine, uint64_t workspace,
                             int64_t workspace_floats, uint64_t stream);

/* Backward of mfh_conv_forward. dy is gated by the fused activation through the forward output y.
 *   db   = FP64 sum of dy per channel: per-tile FP64 partials in `partial` (N * grid_x * CO
 *          doubles, grid_x in [1, ceil(OH*OW / 64)]) reduced in a fixed order;
 *   dw   (CO, CI*KH*KW) = dyT^T cols, dyT (N*OH*OW x CO) being the gated, transposed dy (split-K on
 *          dw_engine through the workspace);
 *   dx   = col2im of grad_cols (N*OH*OW*CI*KH*KW floats), which receives the feature-major column
 *          gradient on dx_engine: W^T dyT^T (CI*KH*KW x N*OH*OW) when dyT is formed (dw requested
 *          or a fused activation), else W^T dy_n (CI*KH*KW x OH*OW) per image from the NCHW dy.
 * dx/grad_cols and partial/db are given together or not at all; dw needs cols and dyT; dx through
 * an activation needs dyT.
 * Replaces mf_conv_backward_plans / mf_conv_backward, native_cublas.cpp:1465-1532. */
MFH_API int mfh_conv_backward(uint64_t weight, uint64_t dy, uint64_t y, uint64_t cols, uint64_t dyT, uint64_t dw,
                              uint64_t grad_cols, uint64_t dx, uint64_t partial, uint64_t db, int N, int CI, int H,
                              int W, int CO, int KH, int KW, int OH, int OW, int SH, int SW, int PH, int PW,
                              int grid_x, int activation, float alpha, int dw_engine, int dx_engine,
                              uint64_t workspace, int64_t workspace_floats, uint64_t stream);

/* mfh_conv_backward with one engine for the dW and the dX products (the same argument list with
 * `engine` in place of dw_engine, dx_engine).
 * Replaces mf_conv_backward, native_cublas.cpp:1523-1532. */
MFH_API int mfh_conv_backward_single(uint64_t weight, uint64_t dy, uint64_t y, uint64_t cols, uint64_t dyT,
                                     uint64_t dw, uint64_t grad_cols, uint64_t dx, uint64_t partial, uint64_t db,
                                     int N, int CI, int H, int W, int CO, int KH, int KW, int OH, int OW, int SH,
                                     int SW, int PH, int PW, int grid_x, int activation, float alpha, int engine,
                                     uint64_t workspace, int64_t workspace_floats, uint64_t stream);

/* Implicit-GEMM convolution forward: y (N,CO,OH,OW) = act(conv(x, weight) + bias [+ residual]) with the im2col
 * matrix gathered from x inside the GEMM's operand loads (no cols buffer). One GEMM
 * W (CO x K) . view (K x N*OH*OW) over every image, stored straight into NCHW with the bias and
 * activation in its epilogue. When CI is a multiple of 32 the features run in channel chunks of 32
 * per window tap and the product reads the kernel in that order from `wt` (CO*CI*KH*KW floats,
 * 16-byte aligned): with prepared = 0 this call writes it there from `weight`; with prepared = 1
 * wt already holds it (mfh_conv_weight_orders, flip 0) and `weight` is not read (it may be 0).
 * Otherwise wt is unused and may be 0. workspace: mfh_conv_implicit_workspace(..., 0) floats let
 * it split K (0 is allowed: no split). engine: 1 (automatic plan) or 16 + tile * 128 + slices - 1
 * over the 12 tiles of the implicit products. residual (may be 0): an NCHW tensor of y's shape added
 * to conv + bias before the activation, each addition rounded to float32 as separate operations
 * would be (the fused Conv + Add + ReLU of an inference graph); it must not overlap y (the call
 * rejects residual == y). Arguments otherwise as
 * mfh_conv_forward.
 * Has no single counterpart in the reference: it replaces the im2col + gemm_rows + epilogue sequence
 * of mf_conv_forward, native_cublas.cpp:1441-1461, when the caller does not keep cols. */
MFH_API int mfh_conv_forward_implicit(uint64_t x, uint64_t weight, uint64_t wt, int prepared, uint64_t bias,
                                      uint64_t residual, uint64_t y, int N, int CI, int H, int W, int CO, int KH, int KW, int OH, int OW,
                                      int SH, int SW, int PH, int PW, int activation, float alpha, int engine,
                                      uint64_t workspace, int64_t workspace_floats, uint64_t stream);

/* mfh_conv_forward_implicit without residual or activation, for a caller that forms y itself:
 * when the product's plan splits K (over the caller's workspace), the product's slices are left in
 * the workspace unreduced (slices x CO x N*OH*OW floats) and *slices receives their count; y is then
 * not written (mfh_bn_forward_split forms it, adding bias (optional, per output channel), and
 * stores it). Otherwise y is written as by
 * mfh_conv_forward_implicit and *slices is 1. No counterpart in the reference: the fused graph's
 * Conv + BN pairs use it. */
MFH_API int mfh_conv_forward_implicit_deferred(uint64_t x, uint64_t weight, uint64_t wt, int prepared, uint64_t bias,
                                               uint64_t y, int N, int CI, int H, int W, int CO, int KH, int KW, int OH, int OW,
                                               int SH, int SW, int PH, int PW, int engine, uint64_t workspace,
                                               int64_t workspace_floats, int* slices, uint64_t stream);

/* The kernels of several convolutions in the orders the implicit products read them, in one
 * launch for up to 32 orders (more take more launches). Kernel i is weights[i] (CO, CI, KH, KW)
 * with dims[9i .. 9i+8] = CO, CI, KH, KW, flip, SH, SW, PH, PW; outs[i] receives CO*CI*KH*KW
 * floats (16-byte aligned): flip 0, the forward order (rows co, features (ci, tap), in chunks of 32
 * channels per tap when CI is a multiple of 32); flip 1, the dX order: for stride 1 the kernel
 * flipped and transposed (rows ci, features (co, KH*KW-1-tap), chunked when CO is a multiple of
 * 32); for larger strides the same for the sub-kernel of each dX phase in turn (phase (a, b) in
 * [0, SH) x [0, SW), a-major: the taps kh = (a+PH)%SH + SH*t, kw = (b+PW)%SW + SW*u, flipped),
 * back to back. Stride and padding matter for the strided dX order only. The three arrays are
 * host memory.
 * Has no counterpart in the reference (its products read the kernel in place): it lets a network
 * reorder all of its kernels once per step instead of once per convolution call. */
MFH_API int mfh_conv_weight_orders(const uint64_t* weights, const uint64_t* outs, const int* dims, int count,
                                   uint64_t stream);

/* Split-K workspace floats of one pass of the implicit convolution under the automatic plan
 * (pass 0 forward, 1 dW, 2 dX of a stride-1 convolution); 0 when it does not split, -1 on error. */
MFH_API int64_t mfh_conv_implicit_workspace(int N, int CI, int H, int W, int CO, int KH, int KW, int OH, int OW,
                                            int SH, int SW, int PH, int PW, int pass);

/* flags of mfh_conv_backward_implicit */
#define MFH_CONV_WFLIP_READY 1   /* wflip already holds the dX order (mfh_conv_weight_orders, flip 1) */
#define MFH_CONV_ACCUMULATE_DX 2 /* dx += the input gradient (dx holds a gradient already) */
#define MFH_CONV_COLUMN_ORDER 4  /* a strided dX through grad_cols reads the column order in wflip */

/* Backward of a convolution without cols, from x and the NCHW dy:
 *   gated (N*CO*OH*OW floats) receives dy gated by the fused activation through y; required when
 *          activation != 0, and then used in place of dy below;
 *   db   = FP64 sum of dy per channel: with dw, the dW product's first feature tile sums dy over
 *          its pixel slice in FP64 (into `partial` when the product is split over the pixels, then
 *          added in slice order by the split-K reduction launch); without dw, per-(n, co) FP64 row
 *          sums reduced over n in order. partial holds CO * max(N, 256) doubles;
 *   dw   (CO, CI*KH*KW) = dy . im2col(x) with dy read in place (split over the pixels on dw_engine
 *          through the workspace); needs x;
 *   dx   with `wflip` (CI*CO*KH*KW floats, 16-byte aligned, the dX order of
 *          mfh_conv_weight_orders for this geometry, which this call fills from `weight` unless
 *          flags has MFH_CONV_WFLIP_READY): stride 1, a forward convolution of dy with the flipped
 *          kernel; larger strides, one such stride-1 convolution of dy with the flipped sub-kernel
 *          of each phase (a, b) (input positions SH*i + a, SW*j + b; the taps that reach them),
 *          each written to its lattice of dx, positions that no tap reaches set to 0; straight
 *          into NCHW dx. Strides above 1 without wflip: the per-image column gradient W^T dy_n in
 *          grad_cols (N*CI*KH*KW*OH*OW floats) and the col2im gather; with grad_cols and
 *          MFH_CONV_COLUMN_ORDER (CO a multiple of 32) the column gradient is one implicit product
 *          over every image, the dX of a 1x1 convolution from CI*KH*KW channels to CO on the OH x OW
 *          grid, whose kernel order wflip holds (mfh_conv_weight_orders of W seen as a
 *          CO x CI*KH*KW x 1 x 1 kernel, flip 1; filled from `weight` here unless
 *          MFH_CONV_WFLIP_READY).
 *          With MFH_CONV_ACCUMULATE_DX, dx = dx + the gradient (one rounding, as a separate add).
 * workspace: at least the larger of mfh_conv_implicit_workspace passes 1 and 2 that are requested
 * (pass 2 covers the largest phase product of a strided dX).
 * dw_engine and the dx_engine of a dX through wflip are implicit plan codes (as
 * mfh_conv_forward_implicit; applied to every phase product); with grad_cols, dx_engine is a GEMM
 * engine code (as mfh_gemm).
 * Has no single counterpart in the reference: it replaces mf_conv_backward_plans,
 * native_cublas.cpp:1465-1532, when the caller does not keep cols. */
MFH_API int mfh_conv_backward_implicit(uint64_t x, uint64_t weight, uint64_t dy, uint64_t y, uint64_t gated,
                                       uint64_t dw, uint64_t dx, uint64_t wflip, uint64_t grad_cols, uint64_t partial,
                                       uint64_t db, int N, int CI, int H, int W, int CO, int KH, int KW, int OH,
                                       int OW, int SH, int SW, int PH, int PW, int activation, float alpha,
                                       int dw_engine, int dx_engine, int flags, uint64_t workspace,
                                       int64_t workspace_floats, uint64_t stream);

/* mfh_conv_backward_implicit with the dW product (and db) on a second stream: dw_stream is first
 * ordered after the work issued so far on `stream` (after the gating of dy, with a fused
 * activation), the dW and db launches go to dw_stream and the dX launches to `stream`, so the two
 * run side by side. The workspace holds the dW part (its first dw_workspace_floats, at least
 * mfh_conv_implicit_workspace pass 1) followed by the dX part (at least pass 2). dw and db are
 * complete once `stream` has been ordered after dw_stream (mfh_stream_wait(stream, dw_stream));
 * every buffer must stay allocated until then. The results are bitwise those of the one-stream call.
 * No counterpart in the reference (one stream per call): for a backward pass that runs the
 * convolutions' dW products beside their dX products. */
MFH_API int mfh_conv_backward_implicit_streams(uint64_t x, uint64_t weight, uint64_t dy, uint64_t y, uint64_t gated,
                                               uint64_t dw, uint64_t dx, uint64_t wflip, uint64_t grad_cols,
                                               uint64_t partial, uint64_t db, int N, int CI, int H, int W, int CO,
                                               int KH, int KW, int OH, int OW, int SH, int SW, int PH, int PW,
                                               int activation, float alpha, int dw_engine, int dx_engine, int flags,
                                               uint64_t workspace, int64_t dw_workspace_floats,
                                               int64_t workspace_floats, uint64_t stream, uint64_t dw_stream);

/* mfh_conv_backward_implicit_streams for a caller that forms dx itself: when the convolution has
 * stride 1, dx is written fresh (no CONV_ACCUMULATE_DX) and the dX product's plan splits K (over the
 * dX part of the workspace, which starts dw_workspace_floats floats in), the product's slices are
 * left there unreduced (slices x CI x N*H*W floats, laid out as mfh_bn_forward_split's partial)
 * and *dx_slices receives their count; dx is then not written (mfh_bn_backward_split forms it and
 * stores it). Otherwise dx is written as by mfh_conv_backward_implicit_streams and *dx_slices is 1.
 * No counterpart in the reference: the fused graph's BN -> Conv pairs use it in the backward. */
MFH_API int mfh_conv_backward_implicit_deferred(uint64_t x, uint64_t weight, uint64_t dy, uint64_t y, uint64_t gated,
                                                uint64_t dw, uint64_t dx, uint64_t wflip, uint64_t grad_cols,
                                                uint64_t partial, uint64_t db, int N, int CI, int H, int W, int CO,
                                                int KH, int KW, int OH, int OW, int SH, int SW, int PH, int PW,
                                                int activation, float alpha, int dw_engine, int dx_engine, int flags,
                                                uint64_t workspace, int64_t dw_workspace_floats,
                                                int64_t workspace_floats, int* dx_slices, uint64_t stream,
                                                uint64_t dw_stream);

/* ---- max pooling ---------------------------------------------------------------------------- */

/* Max-pool without padding (the caller pads with -inf): y = window max in (kh, kw) order with the
 * first maximum winning ties and NaN taking over; argmax (int32) = flat index into x, or 0 when no
 * backward will read it (an inference pass), in which case it is not written.
 * Replaces mf_pool_forward, native_cublas.cpp:1534-1547 (which always writes its mask). */
MFH_API int mfh_pool_forward(uint64_t x, uint64_t y, uint64_t argmax, int N, int C, int H, int W, int OH, int OW,
                             int KH, int KW, int SH, int SW, uint64_t stream);

/* dx[i] = sum of dy over the windows whose argmax is i, in (oh, ow) order.
 * Replaces mf_pool_backward, native_cublas.cpp:1549-1562. */
MFH_API int mfh_pool_backward(uint64_t dy, uint64_t argmax, uint64_t dx, int N, int C, int H, int W, int OH, int OW,
                              int KH, int KW, int SH, int SW, uint64_t stream);

/* ---- GEMM ----------------------------------------------------------------------------------- */

/* C(M,N) = A(M,K) B(K,N) [+ bias(N)], row-major, with a teaching kernel. variant: 0 basic, 1 tiled,
 * 2 shared, 4 register (3, cuBLAS in the reference, is rejected); tile 16/32 for variants 1-2;
 * accumulate: 0 fp32, 1 Kahan-grouped, 2 Dot2. variant 4 with accumulate 0 runs the MFMA engine.
 * Replaces mf_matmul, native_cublas.cpp:1567-1613. */
MFH_API int mfh_matmul(int variant, int tile, int accumulate, uint64_t a, uint64_t b, uint64_t bias, uint64_t c, int M,
                       int N, int K, uint64_t stream);

/* Number of GEMM tiles and their geometry: values[0..4] = BM, BN, WM, WN, BK (block tile, wave
 * tile, LDS stage depth). Replaces mf_gemm_tile_count / mf_gemm_tile_info, native_cublas.cpp:1617-1624
 * (values[2..3] are the wave tile where the reference reports the thread tile). */
MFH_API int mfh_gemm_tile_count(void);
MFH_API int mfh_gemm_tile_info(int index, int* values);

/* K groups of a tile: 1, or the number of wave sets (each of (BM/WM) x (BN/WN) waves) that share
 * the tile's K range in one workgroup, each summing its run of stages, the runs' sums then added
 * in group order; -1 for an unknown tile. No counterpart in the reference (its tiles run one
 * thread set per output tile); a catalogue reader names such tiles apart (e.g. "64x64k4"). */
MFH_API int mfh_gemm_tile_groups(int index);

/* LDS stages a tile's main loop keeps in flight: 2 for every tile (double-buffered operand tiles),
 * or -1 for an unknown tile. Replaces mf_gemm_tile_stages, native_cublas.cpp:1627-1633 (whose
 * 0 meant register double buffering and 2-4 a cp.async pipeline). */
MFH_API int mfh_gemm_tile_stages(int index);

/* Automatic tile and split-K slice count for C(M,N) over K.
 * Replaces mf_gemm_plan, native_cublas.cpp:1635-1643. */
MFH_API int mfh_gemm_plan(int M, int N, int K, int* tile, int* slices);

/* Workspace floats the automatic plan uses (0 when it does not split), -1 on error.
 * Replaces mf_gemm_workspace, native_cublas.cpp:1659-1666. */
MFH_API int64_t mfh_gemm_workspace(int M, int N, int K);

/* C = (float) FP64 sum of slices x M x N contiguous partials in slice order (the split-K
 * reduction); `reference` is accepted for interface parity and selects the same kernel.
 * Replaces mf_split_reduce, native_cublas.cpp:1647-1655. */
MFH_API int mfh_split_reduce(uint64_t partial, uint64_t c, int slices, int M, int N, int ldc, int reference,
                             uint64_t stream);

/* C(M,N) = op(A) op(B) [+ bias(N)], row-major with leading dimensions lda/ldb/ldc. op(A) = A^T when
 * trans_a (A stored K x M), op(B) = B^T when trans_b (B stored N x K); not both. workspace may be
 * 0; with the plan's slices * M * N floats the engine splits K. bias needs ldc == N. Engine 1 with
 * N <= 8 runs one wave per output row (lanes split K, a fixed butterfly adds them); an explicit
 * plan code always runs the MFMA tiles.
 * Replaces mf_gemm, native_cublas.cpp:1672-1692. */
MFH_API int mfh_gemm(int engine, int trans_a, int trans_b, uint64_t a, uint64_t b, uint64_t bias, uint64_t c, int M,
                     int N, int K, int lda, int ldb, int ldc, uint64_t workspace, int64_t workspace_floats,
                     uint64_t stream);

/* Floats of the static split-K scratch of mfh_gemm_noalloc (32 MiB per GPU). */
#define MFH_GEMM_NOALLOC_SCRATCH_FLOATS 8388608

/* mfh_gemm without a workspace argument, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the split-K partials go
 * to a fixed device array inside the library (MFH_GEMM_NOALLOC_SCRATCH_FLOATS floats per GPU, held
 * until the process ends). The call allocates nothing. A plan whose slices * M * N exceeds the
 * scratch is rejected with status 2 (the plan is the one mfh_gemm would run given a large enough
 * workspace: engine 1's automatic plan, or an explicit code). Every call on a GPU shares that GPU's
 * scratch: calls that overlap in time on one GPU (on other streams or threads) race. Results are
 * bitwise those of mfh_gemm with the same engine and a workspace of the plan's size.
 * No counterpart in the reference (its mf_gemm always takes the caller's workspace). */
MFH_API int mfh_gemm_noalloc(int engine, int trans_a, int trans_b, uint64_t a, uint64_t b, uint64_t bias, uint64_t c,
                             int M, int N, int K, int lda, int ldb, int ldc, uint64_t stream);

/* ---- batch normalisation (+ residual add + ReLU) -------------------------------------------- */

/* FP64 workspace (doubles, 16-byte aligned) that mfh_bn_forward (training) and mfh_bn_backward need
 * for an NCHW tensor of N x C x HW elements; -1 on error. No reference counterpart: the reference sizes its
 * partial buffer inline (ops/fused.py:238-243, 265-266). */
MFH_API int64_t mfh_bn_workspace(int N, int C, int HW);

/* Batch norm of x (N, C, HW) per channel. Training: FP64 batch mean / biased variance, mean stored
 * as the float pair mean[c] + mean[C + c], inv_std[c] = 1 / sqrt(var + eps) rounded once, running
 * statistics updated with momentum (the variance scaled by var_scale). Eval: running statistics.
 * y = (((x - mean_hi) - mean_lo) * inv_std) * gamma + beta, then + residual (optional), then ReLU
 * when relu != 0, each operation rounded to float32.
 * Replaces batchnorm2d_forward, ops/fused.py:250-305 (and the BatchNormActivation forward of
 * ops/batchnorm.py:75-94). */
MFH_API int mfh_bn_forward(uint64_t x, uint64_t gamma, uint64_t beta, uint64_t running_mean, uint64_t running_var,
                           uint64_t residual, uint64_t y, uint64_t mean, uint64_t inv_std, uint64_t workspace,
                           int64_t workspace_doubles, int N, int C, int HW, int training, int relu, double momentum,
                           double eps, double var_scale, uint64_t stream);

/* Training mfh_bn_forward of a convolution output that mfh_conv_forward_implicit_deferred left as
 * `slices` FP32 split-K slices (partial: slices x C x N*HW floats, channel c's position
 * n * HW + hw of slice z at partial[(z * C + c) * N * HW + n * HW + hw]). x is formed first, each
 * element the FP64 sum of its slices in slice order rounded once, plus bias[c] (optional) in
 * float32 (the bits of mfh_conv_forward_implicit's own slice reduction), and stored into x; then y, mean, inv_std and the running statistics are those of
 * mfh_bn_forward on that x, in one launch. Only for shapes whose channels are normalised in one
 * launch (N * HW at most 8192); others return status 2. No counterpart in the reference (its
 * convolution and batch norm are separate operators): the fused graph's Conv + BN pairs use it. */
MFH_API int mfh_bn_forward_split(uint64_t partial, int slices, uint64_t bias, uint64_t x, uint64_t gamma, uint64_t beta,
                                 uint64_t running_mean, uint64_t running_var, uint64_t residual, uint64_t y,
                                 uint64_t mean, uint64_t inv_std, int N, int C, int HW, int relu, double momentum,
                                 double eps, double var_scale, uint64_t stream);

/* Gradients of mfh_bn_forward. g = dy, or dy where gate > 0 and 0 elsewhere when gate (the fused
 * ReLU's output) is given; residual_grad (optional, needs gate) receives g. dgamma / dbeta are
 * FP64 sums; x_grad = a * ((g - k1) - ((x - mean_hi) - mean_lo) * k2) in training,
 * a * g in eval, with a = gamma * inv_std, k1 = sum(g) / count, k2 = inv_std * dgamma / count.
 * Each output is stored, or added when its add_* flag is set.
 * Replaces batchnorm2d_backward, ops/fused.py:308-380. */
MFH_API int mfh_bn_backward(uint64_t x, uint64_t dy, uint64_t gate, uint64_t gamma, uint64_t mean, uint64_t inv_std,
                            uint64_t x_grad, uint64_t gamma_grad, uint64_t beta_grad, uint64_t residual_grad,
                            uint64_t workspace, int64_t workspace_doubles, int N, int C, int HW, int training,
                            int add_x, int add_gamma, int add_beta, int add_residual, uint64_t stream);

/* mfh_bn_backward whose dy is the dx of a convolution that mfh_conv_backward_implicit_deferred left
 * as `slices` FP32 split-K slices (partial laid out as in mfh_bn_forward_split): dy is formed first,
 * each element the FP64 sum of its slices in slice order rounded once (the bits of the product's
 * own slice reduction), and stored into dy; then the gradients are those of mfh_bn_backward on that
 * dy, in one launch. Only for passes that sum over one launch per channel (N * HW at most 8192, a
 * gradient of gamma, beta or, in training, x asked for); others return status 2. No counterpart in
 * the reference (its convolution and batch norm are separate operators): the fused graph's
 * BN -> Conv pairs use it. */
MFH_API int mfh_bn_backward_split(uint64_t partial, int slices, uint64_t x, uint64_t dy, uint64_t gate, uint64_t gamma,
                                  uint64_t mean, uint64_t inv_std, uint64_t x_grad, uint64_t gamma_grad,
                                  uint64_t beta_grad, uint64_t residual_grad, uint64_t workspace,
                                  int64_t workspace_doubles, int N, int C, int HW, int training, int add_x,
                                  int add_gamma, int add_beta, int add_residual, uint64_t stream);

/* Batch norm + ReLU + max-pool (KH x KW window, stride SH x SW, no padding) as one unit, for a
 * network stem: the ReLU output is never stored. Returns 1 when the fused kernels take this shape
 * (their LDS staging of a plane fits), else 0.
 * No counterpart in the reference (there, BatchNormActivation's output feeds MaxPool2d_Op):
 * it spares the ReLU output's HBM round trip and the max-pool's passes. */
MFH_API int mfh_bn_relu_pool_supported(int N, int C, int H, int W, int KH, int KW, int SH, int SW);

/* mfh_bn_forward with relu (no residual) followed by mfh_pool_forward on its output: pooled and
 * argmax (N, C, OH, OW) with OH = (H - KH) / SH + 1, argmax the int32 flat index into the
 * N x C x H x W tensor. mean / inv_std / running statistics and workspace as mfh_bn_forward.
 * The same bits as those two calls. */
MFH_API int mfh_bn_relu_pool_forward(uint64_t x, uint64_t gamma, uint64_t beta, uint64_t running_mean,
                                     uint64_t running_var, uint64_t pooled, uint64_t argmax, uint64_t mean,
                                     uint64_t inv_std, uint64_t workspace, int64_t workspace_doubles, int N, int C,
                                     int H, int W, int KH, int KW, int SH, int SW, int training, double momentum,
                                     double eps, double var_scale, uint64_t stream);

/* The unit's backward from the pooled gradient: mfh_pool_backward into the ReLU output's gradient,
 * gated by the ReLU (recomputed from x, mean, inv_std, gamma and beta), then mfh_bn_backward, with
 * the same bits and add_* flags; nothing of the ReLU output's size is written but x_grad. */
MFH_API int mfh_bn_relu_pool_backward(uint64_t x, uint64_t pooled_grad, uint64_t argmax, uint64_t gamma,
                                      uint64_t beta, uint64_t mean, uint64_t inv_std, uint64_t x_grad,
                                      uint64_t gamma_grad, uint64_t beta_grad, uint64_t workspace,
                                      int64_t workspace_doubles, int N, int C, int H, int W, int KH, int KW, int SH,
                                      int SW, int training, int add_x, int add_gamma, int add_beta, uint64_t stream);

/* ---- activations and the optimiser ---------------------------------------------------------- */

/* y = max(0, x) over count elements (NaN stays NaN).
 * Replaces the forward of ReLU, ops/activation.py:43-48. */
MFH_API int mfh_relu_forward(uint64_t x, uint64_t y, int64_t count, uint64_t stream);

/* out = (x > 0 ? grad : alpha * grad), or out += that when add != 0 (alpha = 0: ReLU).
 * Replaces relu_backward_accumulate / leaky_relu_backward_accumulate, ops/fused.py:50-77. */
MFH_API int mfh_relu_backward(uint64_t x, uint64_t grad, uint64_t out, int64_t count, float alpha, int add,
                              uint64_t stream);

/* ---- head and loss ---------------------------------------------------------------------------- */

/* y[p] = float(FP64 sum of x[p*hw .. p*hw + hw) / hw) for `planes` contiguous planes of hw floats:
 * the global average pool of an NCHW tensor (planes = N*C, hw = H*W).
 * Replaces GlobalAvgPool2d_Op.forward, ops/batchnorm.py:113-116. */
MFH_API int mfh_plane_mean(uint64_t x, uint64_t y, int64_t planes, int hw, uint64_t stream);

/* dx[p*hw + i] = dy[p] / float(hw), or dx += that when add != 0.
 * Replaces GlobalAvgPool2d_Op.backward, ops/batchnorm.py:118-123 (the broadcast gradient written out). */
MFH_API int mfh_plane_mean_backward(uint64_t dy, uint64_t dx, int64_t planes, int hw, int add, uint64_t stream);

/* loss[0] = float(FP64 sum of float32 (pred - target)^2 / count) (count = 0: NaN, the mean of nothing).
 * Replaces MSELoss.forward, ops/loss.py:99-106. */
MFH_API int mfh_mse_loss(uint64_t pred, uint64_t target, uint64_t loss, int64_t count, uint64_t stream);

/* grad = seed[0] * ((2 * (pred - target)) / float(count)), each operation rounded to float32, or
 * grad += that when add != 0 (seed: the loss gradient, one float on the device).
 * Replaces MSELoss.backward, ops/loss.py:108-113. */
MFH_API int mfh_mse_loss_backward(uint64_t pred, uint64_t target, uint64_t seed, uint64_t grad, int64_t count, int add,
                                  uint64_t stream);

/* out[j] = float(FP64 sum over r < rows of src[r*cols + j]): a Linear layer's bias gradient.
 * Replaces _reduce_to(grad, b.shape) in Linear.backward, ops/basic.py:164. */
MFH_API int mfh_column_sums(uint64_t src, uint64_t out, int64_t rows, int64_t cols, uint64_t stream);

/* One tensor of an Adam step: parameter, gradient and moments (size floats each, contiguous), the
 * learning rate, the weight decay and the bias corrections 1 - beta1^step, 1 - beta2^step, all
 * rounded to float32. */
typedef struct mfh_adam_tensor {
    uint64_t param, grad, m, v;
    int64_t size;
    float lr, weight_decay, bias_correction1, bias_correction2;
} mfh_adam_tensor;

/* Adam over `count` tensors (the table is host memory, read during the call):
 * m = b1 m + (1 - b1) gs; v = b2 v + (1 - b2) gs^2; p -= (lr (m / bc1)) / (sqrt(v / bc2) + eps),
 * gs = g * grad_scale (+ weight_decay * p), every operation rounded to float32 in that order.
 * Replaces adam_update / adam_update_many, ops/fused.py:514-533 and 609-621. */
MFH_API int mfh_adam_step(const mfh_adam_tensor* tensors, int count, float grad_scale, float beta1,
                          float one_minus_beta1, float beta2, float one_minus_beta2, float eps, uint64_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MFHIP_H */
