/*
 * lava_hip.h -- C ABI of liblava_hip.so, the MI355X (gfx950) implementation of
 * Lava.jl's cooperative-matrix compute path.
 *
 * Conventions for every entry point:
 *   - returns LAVA_HIP_OK (0) on success, a negative status otherwise; the
 *     thread-local message is read with lava_hip_last_error().  No exception
 *     crosses the ABI.
 *   - pointers to device memory are plain addresses (hipMalloc'd or any other
 *     device allocation); the caller owns every buffer.
 *   - `stream` is a hipStream_t passed as void*; NULL is the default (NULL) stream.
 *     Launches are asynchronous on that stream.  lava_hip_stream_create makes a
 *     NON-BLOCKING stream (hipStreamNonBlocking): it is not ordered after work on
 *     the NULL stream, so a caller that fills inputs on the NULL stream synchronises
 *     (lava_hip_synchronize, or an event) before launching on it.
 *   - element strides (lda, ldb, ...) are in elements, not bytes.
 *   - argument checks happen on the host before any GPU call, so a bad call
 *     fails with LAVA_HIP_ERR_INVALID_ARG / _UNSUPPORTED and touches no device.
 *
 * Reference boundary being replaced (Lava.jl, paths relative to its tree):
 * Lava compiles a kernel written against the vocabulary of
 * src/vocabulary/coopmat.jl into a `LavaGPUKernel` (src/compiler/compilation.jl:409-426,
 * src/compiler/cache.jl:109-138) whose arguments travel in one buffer addressed by
 * an 8-byte push constant (src/compiler/entry_wrapper.jl:26-178); the launcher
 * (Mantle.jl) dispatches it.  Here each kernel is compiled ahead of time and each
 * entry point takes its arguments directly.
 */
#ifndef LAVA_HIP_H
#define LAVA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
#define LAVA_HIP_OK 0
#define LAVA_HIP_ERR_INVALID_ARG (-1) /* shape, stride, pointer or alignment error */
#define LAVA_HIP_ERR_UNSUPPORTED (-2) /* valid request this build does not implement */
#define LAVA_HIP_ERR_HIP (-3)         /* the HIP runtime reported an error */
#define LAVA_HIP_ERR_NO_DEVICE (-4)   /* no usable gfx950 device */

/* ---- element type codes (dtype arguments) ------------------------------- */
#define LAVA_HIP_F16 0
#define LAVA_HIP_BF16 1
#define LAVA_HIP_F32 2
#define LAVA_HIP_I8 3
#define LAVA_HIP_U8 4
#define LAVA_HIP_I32 5
#define LAVA_HIP_U32 6
#define LAVA_HIP_F64 7

/* ---- GEMM layout flags ---------------------------------------------------
 * bit0: A row-major, bit1: B row-major, bit2: C row-major; a clear bit means
 * column-major, Julia's default (src/device/devicearray.jl:138-174).  Row- vs
 * column-major is the MemoryLayout operand of the load/store
 * (src/vocabulary/coopmat.jl:124-161; src/compiler/spirv/coopmat.jl:664-744). */
#define LAVA_HIP_A_ROWMAJOR 1u
#define LAVA_HIP_B_ROWMAJOR 2u
#define LAVA_HIP_C_ROWMAJOR 4u

/* ---- CoopMatReduce masks (src/vocabulary/coopmat.jl:292-297) ------------- */
#define LAVA_HIP_REDUCE_ROW 1u
#define LAVA_HIP_REDUCE_COLUMN 2u
#define LAVA_HIP_REDUCE_ROW_AND_COLUMN 3u
#define LAVA_HIP_REDUCE_TWO_BY_TWO 4u /* 2 x 2 blocks (lava_hip_coopmat_reduce_into); unverified in the reference */

/* reduce combiners */
#define LAVA_HIP_COMBINE_ADD 0
#define LAVA_HIP_COMBINE_MAX 1
#define LAVA_HIP_COMBINE_MIN 2

/* ========================================================================= */
/* Runtime plumbing: what Mantle's LavaArray / buffer layer provides to a     */
/* Lava kernel (README.md:11-13), reduced to hipMalloc/hipMemcpy wrappers.    */
/* ========================================================================= */

/* Idempotent and thread-safe.  Selects nothing; checks that device 0 is gfx950.
 * Replaces the device/context set-up Lava leaves to Mantle (src/Lava.jl:128-142). */
int lava_hip_init(void);
int lava_hip_device_count(int* count);
int lava_hip_malloc(void** ptr, size_t bytes);
int lava_hip_free(void* ptr);
int lava_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int lava_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);
/* Device-to-device copy by a kernel (graph-capture safe), asynchronous on `stream`. */
int lava_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* Byte fill by a kernel (not hipMemsetAsync), so it is safe under graph capture. */
int lava_hip_fill_bytes(void* dst, uint8_t value, size_t bytes, void* stream);
int lava_hip_synchronize(void);
int lava_hip_stream_synchronize(void* stream);
/* A non-blocking stream (hipStreamNonBlocking, default priority). */
int lava_hip_stream_create(void** stream);
/* Waits for the stream's work, frees the workspace the library kept for it (W8A16 and
 * small-product GEMM split-K; buffers a graph captured on the stream may still use are kept
 * until the process ends), then destroys it. */
int lava_hip_stream_destroy(void* stream);
int lava_hip_event_create(void** event);
int lava_hip_event_destroy(void* event);
int lava_hip_event_record(void* event, void* stream);
int lava_hip_event_elapsed_ms(float* ms, void* start, void* stop);
/* HIP graphs of the library's calls (thin wrappers over hipStreamBeginCapture in global mode,
 * hipStreamEndCapture + hipGraphInstantiate, hipGraphLaunch, hipGraphExecDestroy): what a caller
 * that replays a fixed sequence of launches uses instead of a tracing compiler.  While a stream
 * captures in global mode, an allocating call anywhere in the process fails; the compute entry
 * points then plan within the workspace the stream already has (lava_hip_gemm_w8a16) or take
 * lava_hip_gemm_w8a16_noalloc.  The NULL stream cannot be captured. */
int lava_hip_graph_capture_begin(void* stream);
int lava_hip_graph_capture_end(void* stream, void** exec);
int lava_hip_graph_launch(void* exec, void* stream);
int lava_hip_graph_destroy(void* exec);
/* Thread-local message of the last failure on this thread ("" if none).
 * Replaces LavaError/LavaCompilationError reporting (src/runtime/errors.jl:12-51). */
const char* lava_hip_last_error(void);
/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int lava_hip_version(void);
/* Frees every workspace the library keeps (W8A16 split-K partials or the row-major copy of X,
 * small-product GEMM split-K partials), after waiting for each device that holds one
 * (hipDeviceSynchronize): the release path of the NULL stream's workspaces, which
 * lava_hip_stream_destroy does not reach, and of streams created outside the library.  Buffers
 * that a graph captured on a stream may still use are kept until the process ends.  No
 * counterpart in the reference (Lava owns no memory); the next call that needs a workspace
 * allocates one again. */
int lava_hip_release_workspaces(void);

/* ========================================================================= */
/* Diagnostics (no counterpart in the reference): which kernels a call ran,   */
/* and a kernel choice pinned for tests and A/B measurements.                */
/* ========================================================================= */

/* The names of the kernels this thread launched since its last lava_hip_kernel_log_clear(),
 * '+'-separated, the newest last (at most 255 bytes; the oldest names are dropped first). */
const char* lava_hip_kernel_log(void);
void lava_hip_kernel_log_clear(void);

/* Pins, process-wide, the kernel a family's dispatcher picks (choice 0 restores the automatic
 * choice).  A pinned kernel that cannot take a call's shape or layout is passed over for the
 * automatic choice.  Families and choices:
 *  LAVA_HIP_FAMILY_ATTN: 3 flash_fwd3_kernel (D = 64 or 128, scale > 0), 5 flash_fwd5_kernel
 *                        (D <= 128, a multiple of 8, any scale);
 *  LAVA_HIP_FAMILY_GEMM: 1 the 256 x 256 tile kernel, 2 the 64 x 64 small-product kernel
 *                        without a K split, 3 the staged kernel, 4 the 128 x 128 mid-size kernel
 *                        (f16 / bf16 / int8 / unsigned bytes, any operand layout; the fused
 *                        epilogue for f16 / bf16).
 * Unknown families or choices return LAVA_HIP_ERR_INVALID_ARG. */
/* Reads [src, src + bytes) once with 16-byte nontemporal loads, `unroll` (4, 8 or 16) in flight
 * per thread, `blocks` workgroups of 256 threads, and writes the XOR of what each thread read to
 * sink[thread] (sink holds blocks * 256 words): the HBM read bandwidth the part sustains, the
 * ceiling the W8A16 weight stream is measured against.  src 16-byte aligned, bytes a multiple
 * of 16. */
int lava_hip_read_stream(const void* src, size_t bytes, uint32_t* sink, int blocks, int unroll, void* stream);

/* MFMA forms for lava_hip_mfma_loop. */
#define LAVA_HIP_MFMA_F16_16X16X32 0
#define LAVA_HIP_MFMA_BF16_16X16X32 1
#define LAVA_HIP_MFMA_I8_16X16X64 2
#define LAVA_HIP_MFMA_F16_32X32X16 3
#define LAVA_HIP_MFMA_BF16_32X32X16 4
#define LAVA_HIP_MFMA_I8_32X32X32 5
/* Issues MFMAs of form `op` with no memory access in the loop: `blocks` workgroups of
 * 256 * waves_per_simd (1, 2 or 4) threads, one workgroup per CU at a time, each lane holding four (a, b) operand pairs of 16
 * bytes read once from a and b (lane i takes 16-byte words 4i .. 4i+3, modulo bytes / 16), then
 * `iters` rounds of 16 independent MFMAs of a 16x16 form or 4 of a 32x32 form.  Writes a hash of
 * each thread's accumulators to sink[thread] (blocks * 256 * waves_per_simd floats).  Each wave
 * does iters rounds of 8192 * K FLOP (integer ops for int8; K the form's depth: 32 or 64 for the
 * 16x16 forms, 16 or 32 for the 32x32 forms), blocks * 4 * waves_per_simd waves: the matrix-core
 * rate the part sustains on that data at the clock its power budget allows.  a, b 16-byte
 * aligned, bytes a positive multiple of 16. */
int lava_hip_mfma_loop(int op, const void* a, const void* b, size_t bytes, int blocks, int waves_per_simd,
                       int iters, float* sink, void* stream);

#define LAVA_HIP_FAMILY_ATTN 1
#define LAVA_HIP_FAMILY_GEMM 2
int lava_hip_set_kernel_override(int family, int choice);

/* ========================================================================= */
/* Device capabilities: the MI355X answer to `caps(backend)::DeviceCaps`       */
/* (src/vocabulary/caps.jl:54-170) and `matrix_shapes` (caps.jl:158-159).     */
/* ========================================================================= */

/* out[0..n) receives, in order: coopmat (1), tile (16), subgroup (64),
 * coopmatsubgroup (64), sharedbudget (LDS bytes per workgroup), workgrouplimit,
 * cores (compute units), warps (SIMDs per CU x max waves per SIMD), clock_khz,
 * hbm_bytes, l2_bytes, gfx_arch_number (950).  Fields past n are not written. */
int lava_hip_device_caps(int64_t* out, int n);

/* The subgroup-scope MatrixShape table (src/vocabulary/matrix.jl:88-95): row i is
 * out[6*i .. 6*i+6) = {ab_dtype, acc_dtype, M, N, K, scope(0 = subgroup)}.
 * *count receives the number of rows; at most max_rows are written. */
int lava_hip_matrix_shapes(int32_t* out, int max_rows, int* count);

/* ========================================================================= */
/* Seeded input generator (device side of the oracle's definition)           */
/* ========================================================================= */

/* splitmix64 of (seed, index): uniform[a,b] rounded once to fp32 then RNE to
 * dtype (F16, BF16 or F32). */
int lava_hip_fill_uniform(void* dst, int dtype, int64_t n, uint64_t seed, double a, double b, void* stream);
/* Box-Muller normal(0,1) from one draw per element, fp32 then RNE to dtype. */
int lava_hip_fill_normal(void* dst, int dtype, int64_t n, uint64_t seed, void* stream);
/* int8 over [-128,127] (symmetric=0) or [-127,127] (symmetric=1). */
int lava_hip_fill_i8(void* dst, int64_t n, uint64_t seed, int symmetric, void* stream);

/* ========================================================================= */
/* Tile-level vocabulary: one subgroup (wavefront) per tile                   */
/* ========================================================================= */

/* D = muladd(A, B, C) on 16x16x16 tiles, exactly the sequence
 *   a = AcceleratedMatrix{Ta,16,16,MatrixA}(pA, offA, strideA[, Val(true)])
 *   b = AcceleratedMatrix{Tb,16,16,MatrixB}(pB, offB, strideB[, Val(true)])
 *   c = AcceleratedMatrix{Tc,16,16,Accumulator}(pC, offC, strideC[, Val(true)])
 *   copyto!(pD, offD, strideD, muladd(a, b, c)[, Val(true)])
 * (docs/src/device.md:81-88; src/vocabulary/coopmat.jl:124-161,196-199).
 * Offsets are Lava's 1-based element offsets; strides are element strides
 * between columns (column-major) or rows (row-major).  `layout` bits 0..3 mark
 * A, B, C, D row-major.  `ntiles` independent tiles are processed, tile t
 * reading at offsets + t * tile_step (elements).
 * Type pairs (ab_dtype, acc_dtype): (F16, F32), (I8, I32) signed, (U8, U32)
 * unsigned (test/spirv/test_coopmat_int8.jl:25-98), and the wide component types of the
 * reference's coopmat table (src/device/coopmat_intrinsics.jl:16-19): (F32, F32) on four
 * v_mfma_f32_16x16x4_f32 and (F64, F64) on four v_mfma_f64_16x16x4_f64 per tile. */
int lava_hip_coopmat_muladd_16x16x16(int ab_dtype, int acc_dtype, const void* A, int64_t offA, int64_t strideA,
                                     const void* B, int64_t offB, int64_t strideB, const void* C, int64_t offC,
                                     int64_t strideC, void* D, int64_t offD, int64_t strideD, uint32_t layout,
                                     int64_t ntiles, int64_t tile_step, void* stream);

/* coopmat_perelement(f, m) with f(row, col, e) = e * (row + 1) + col on fp32
 * 16x16 (and 32x32 when tile == 32) Accumulator tiles loaded column-major with
 * stride `tile` from `in` and stored the same way to `out`
 * (test/spirv/test_coopmat_perelement_inline.jl:19-37;
 * src/device/coopmat_intrinsics.jl:535-628). */
int lava_hip_coopmat_perelement_rowcol(const float* in, float* out, int tile, int64_t ntiles, void* stream);

/* coopmat_perelement(f, m, o) with f(row, col, x, y) = max(x, y) + row - col: the
 * matrix-operand form (src/device/coopmat_intrinsics.jl:630-678). */
int lava_hip_coopmat_perelement_pair(const float* m, const float* o, float* out, int tile, int64_t ntiles,
                                     void* stream);

/* coopmat_reduce(f, Dst, m, Val(mask)) on fp32 tile x tile Accumulators (tile 16
 * or 32), same-shape destination, result smeared along the reduced axis
 * (src/device/coopmat_intrinsics.jl:685-755).  combine: LAVA_HIP_COMBINE_*. */
int lava_hip_coopmat_reduce(const float* in, float* out, int tile, uint32_t mask, int combine, int64_t ntiles,
                            void* stream);

/* coopmat_reduce into a destination of another extent -- coopmat2's flexible dimensions, which
 * the reference's flash form uses to resize a Br x Bc matrix to Br x HSV_pad with
 * smearReduce(x, y) = x (src/device/coopmat_intrinsics.jl:685-720;
 * src/vocabulary/coopmat.jl:289-312).  m: fp32 tile x tile Accumulators (tile 16 or 32);
 * Dst: fp32 dst_rows x dst_cols; both column-major in memory, ntiles of each consecutive.
 *   Row (1):          dst_rows == tile, dst_cols 16, 32 or 64: Dst[r][c] = combination of row r;
 *   Column (2):       dst_cols == tile, dst_rows 16, 32 or 64: Dst[r][c] = combination of column c;
 *   RowAndColumn (3): dst_rows, dst_cols 16, 32 or 64: every element the combination of all of m;
 *   TwoByTwo (4):     dst = tile / 2 x tile / 2, Dst[i][j] = f(f(m[2i][2j], m[2i][2j+1]),
 *                     f(m[2i+1][2j], m[2i+1][2j+1])), the 2 x 2 block reduce of the published
 *                     SPV_NV_cooperative_matrix2 extension, in that order (the reference declares
 *                     the bit, src/vocabulary/coopmat.jl:289-297, and calls it unverified).
 * Other destination shapes return LAVA_HIP_ERR_INVALID_ARG. */
int lava_hip_coopmat_reduce_into(const float* in, float* out, int tile, int dst_rows, int dst_cols, uint32_t mask,
                                 int combine, int64_t ntiles, void* stream);

/* convert(AcceleratedMatrix{T,...}, m) of fp32 tiles to F16 or BF16, RNE
 * (src/vocabulary/coopmat.jl:178-182; src/compiler/passes/exact_narrowing.jl:31-36).
 * n must be a multiple of 256 (whole 16x16 tiles). */
int lava_hip_coopmat_convert(const float* in, void* out, int out_dtype, int64_t n, void* stream);

/* Matrix uses (src/vocabulary/matrix.jl:37-46) */
#define LAVA_HIP_USE_MATRIX_A 0
#define LAVA_HIP_USE_MATRIX_B 1
#define LAVA_HIP_USE_ACCUMULATOR 2

/* convert(CoopMatrix{To,T,T,Use}, m) of fp32 tile x tile Accumulators (tile 16 or 32,
 * column-major with stride `tile`, ntiles consecutive tiles) to F16 or BF16 (RNE) *and*
 * to another use: the result is stored column-major through the destination use's lane
 * map, so `out` equals the narrowed input exactly when each element reached the lane
 * that use assigns to it.  Replaces coopmat_convert with a use change (OpFConvert, then
 * OpCooperativeMatrixConvertNV: src/device/coopmat_intrinsics.jl:222-247;
 * src/compiler/spirv/coopmat.jl:783-824). */
int lava_hip_coopmat_convert_use(const float* in, void* out, int out_dtype, int tile, int use, int64_t ntiles,
                                 void* stream);

/* Attention's second product on 16x16x16 tiles: D = convert(MatrixA f16, P) * V + 0, with P
 * an fp32 Accumulator and V an fp16 MatrixB, all column-major with stride 16, ntiles
 * consecutive tiles (the P_A step of flash_attn_cm2, coopmat_intrinsics.jl:222-231). */
int lava_hip_coopmat_convert_use_muladd_16x16x16(const float* P, const void* V, float* D, int64_t ntiles,
                                                 void* stream);

/* D = mul(a, b) or add(a, b) (OpFMul / OpFAdd component-wise, src/compiler/spirv/coopmat.jl:
 * 870-885; src/device/coopmat_intrinsics.jl:402-464) on fp32 tile x tile Accumulators loaded
 * like coopmat_load: strides are element strides between columns (column-major) or rows
 * (row-major); a stride of 0 loads the broadcast factor matrix (every column, or row,
 * reading the same vector).  layout bits 0..2: A, B, D row-major; tile t at + t*tile_step. */
#define LAVA_HIP_ELEMENTWISE_MUL 0
#define LAVA_HIP_ELEMENTWISE_ADD 1
int lava_hip_coopmat_elementwise(int op, int tile, const float* A, int64_t strideA, const float* B, int64_t strideB,
                                 float* D, int64_t strideD, uint32_t layout, int64_t ntiles, int64_t tile_step,
                                 void* stream);

/* `accinit` then muladd on 16x16x16 tiles: c = add(bias at stride 0, residual at ldr);
 * D = muladd(a, b, c).  A, B fp16 16x16 column-major (stride 16) at t*256; bias: 16 fp32
 * per tile (one per row) at t*16; residual and D fp32 column-major, tile t at t*16*ld
 * (src/device/coopmat_intrinsics.jl:435-464). */
int lava_hip_coopmat_accinit_muladd_16x16x16(const void* A, const void* B, const float* bias, const float* residual,
                                             int64_t ldr, float* D, int64_t ldd, int64_t ntiles, void* stream);

/* The portable elementwise epilogue: for i in 0:coopmat_length(m)-1,
 * m = coopmat_setcomp(m, i, act(coopmat_getcomp(m, i))) on fp32 tile x tile Accumulators
 * (column-major, stride tile); *length_out (device memory) receives coopmat_length as the
 * kernel saw it (src/device/coopmat_intrinsics.jl:322-400; coopmat.jl:826-868).
 * act: LAVA_HIP_ACT_* below. */
int lava_hip_coopmat_foreach_act(const float* in, float* out, int tile, int act, int64_t ntiles, int32_t* length_out,
                                 void* stream);

/* coopmat_length(CoopMatrix{dtype,rows,cols,use}) of the fragment types the kernels use:
 * rows * cols / 64 components per lane (host query, no device needed). */
int lava_hip_coopmat_length(int dtype, int rows, int cols, int use, int32_t* length_out);

/* coopmat_perelement(f, m, ptr, base) with a pointer and an offset in `extras`
 * (src/device/coopmat_intrinsics.jl:569-572, 595-628) on fp32 tile x tile Accumulators:
 *   by_row == 0: f(r, c, e, s, b) = e * float(s[b + c]), s fp16 -- the W8A16 dequant scale;
 *   by_row != 0: f(r, c, e, cs, b) = e * cs[b + r], cs fp32 -- attention's row rescale.
 * Tile t passes b = base + t * tile. */
int lava_hip_coopmat_perelement_scale(const float* in, float* out, int tile, int by_row, const void* factors,
                                      int64_t base, int64_t ntiles, void* stream);

/* The workgroup-scope table `wggran` (src/vocabulary/caps.jl:122-145): row i is
 * out[4*i .. 4*i+4) = {invocations, M, N, K}, the multiples a workgroup-scope fp16 x fp16
 * -> fp32 matrix must be at a workgroup of that many invocations. */
int lava_hip_workgroup_shapes(int32_t* out, int max_rows, int* count);

/* C (M x N, fp32) = A (M x K, fp16) * B (K x N, fp16) as ONE workgroup-scope matrix held by
 * a single workgroup of `invocations` lanes (a row of lava_hip_workgroup_shapes); M, N, K
 * must be positive multiples of that row's (M, N, K), at most 4096 each.  layout bits as
 * for the GEMMs below (WorkgroupMatrix, src/vocabulary/coopmat.jl:36-92). */
int lava_hip_coopmat_workgroup_gemm_f16(int invocations, const void* A, const void* B, float* C, int64_t M, int64_t N,
                                        int64_t K, int64_t lda, int64_t ldb, int64_t ldc, uint32_t layout,
                                        void* stream);

/* y[i] = dot4x8(a[i], b[i]) (src/vocabulary/vocabulary.jl:31-35). */
int lava_hip_dot4x8(const uint32_t* a, const uint32_t* b, int32_t* y, int64_t n, void* stream);

/* ---- tensor addressing (src/vocabulary/tensor.jl:1-115; lowered in
 * src/device/tensor_intrinsics.jl) ---- */
/* Clamp modes, the values of TENSOR_CLAMP_UNDEFINED / _CONSTANT / _TO_EDGE (tensor.jl:44-51). */
#define LAVA_HIP_CLAMP_UNDEFINED 0u
#define LAVA_HIP_CLAMP_CONSTANT 1u
#define LAVA_HIP_CLAMP_TO_EDGE 2u

/* A TensorLayout as plain data: what tensor_layout(Val(rank), Val(clamp)) followed by
 * tensor_setdim, tensor_setstride, tensor_setclampvalue and tensor_slice builds
 * (tensor.jl:52-93).  Arrays are outermost first, innermost last, first `rank` entries
 * used.  dim: extents; stride: element strides (a packed tensor has stride[rank-1] = 1);
 * off / size: the slice, 0-based (off may be negative); clampbits: the clamp constant's
 * bits in the matrix's component type, zero-extended (tensor_clampbits, tensor.jl:83-85).
 * The matrix's (row, col) is the slice's coordinate in the last two dimensions; outer
 * dimensions must have slice size 1. */
typedef struct lava_hip_tensor_layout {
    int32_t rank;
    uint32_t clamp;
    uint32_t clampbits;
    int32_t dim[4];
    int32_t stride[4];
    int32_t off[4];
    int32_t size[4];
} lava_hip_tensor_layout;

/* Fragment shapes of the tile entry points (MatrixA R x K, MatrixB K x C, Accumulator). */
#define LAVA_HIP_TILE_A_16x16 0
#define LAVA_HIP_TILE_B_16x16 1
#define LAVA_HIP_TILE_ACC_16x16 2
#define LAVA_HIP_TILE_ACC_32x32 3
#define LAVA_HIP_TILE_A_32x16 4
#define LAVA_HIP_TILE_B_16x32 5

/* m = tensor_load(object, src, layout[, view]) on one fragment, then stored row-major to
 * `out` (R x C, dtype LAVA_HIP_F16 or LAVA_HIP_F32).  `object` (R x C, row-major) is the
 * matrix whose values elements outside the slice keep; elements inside the slice but
 * outside the tensor read the clamp constant (CONSTANT), the nearest element (TO_EDGE),
 * or keep the object's value (UNDEFINED).  transpose != 0 loads through the (1, 0) TensorView.
 * Replaces lava_tensor_load (src/device/tensor_intrinsics.jl:258-320) and KernelInterface's
 * tensor_load (tensor.jl:98-105). */
int lava_hip_tensor_load_tile(int dtype, int shape, const void* src, const lava_hip_tensor_layout* layout,
                              int transpose, const void* object, void* out, void* stream);

/* tensor_store(m, dst, layout[, view]) of the fragment read row-major from `in`: only
 * elements inside both the slice and the tensor are written (the clamping store,
 * src/device/tensor_intrinsics.jl:329-402; tensor.jl:107-108). */
int lava_hip_tensor_store_tile(int dtype, int shape, const void* in, void* dst, const lava_hip_tensor_layout* layout,
                               int transpose, void* stream);

/* D (16 x 16 fp32, row-major) = A * B, with A (fp16 MatrixA 16x16) and B (fp16 MatrixB
 * 16x16) loaded through layouts (B optionally through the transposing view).  With B's
 * layout TENSOR_CLAMP_CONSTANT and a clamp value of one, the columns of B past the tensor
 * read one and those columns of D are the row sums of A: the attention V-padding trick of
 * src/device/tensor_intrinsics.jl:139-155. */
int lava_hip_tensor_muladd_16x16x16(const void* A, const lava_hip_tensor_layout* layout_a, const void* B,
                                    const lava_hip_tensor_layout* layout_b, int transpose_b, float* D, void* stream);

/* ========================================================================= */
/* Kernels                                                                    */
/* ========================================================================= */

/* C (M x N) = A (M x K) * B (K x N), fp32 accumulate, C overwritten.
 * Replaces the coopmat GEMM kernels Lava compiles for Mantle (`coopmat_gemm_kernel!`,
 * named at src/device/coopmat_intrinsics.jl:90; the staged form
 * src/device/coopmat_intrinsics.jl:104-148; the coopmat2 form
 * test/glsl/coopmat2_gemm_regs.comp:37-84 with push block {pa, pb, pc, M, N, K}).
 * Any M, N, K >= 0; layout flags as above; lda/ldb/ldc >= the extent they stride.
 * A product of at most 256 64 x 64 tiles with a long K (at least 8 K chunks of 512 bytes, 16
 * above 128 tiles) splits K: partial products go to the per-stream workspace described at
 * lava_hip_gemm_w8a16 (allocated or grown on first use, same locking and lifetime) and are
 * summed in a fixed order, so repeat calls give the same bits.  These are the only plain-GEMM
 * shapes that allocate; under graph capture they split only within the workspace the stream
 * already has, and run unsplit otherwise. */
int lava_hip_gemm_f16_f32(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                          int64_t ldb, int64_t ldc, uint32_t layout, void* stream);
/* The bf16 form (no Lava counterpart: the coopmat component table has no bf16,
 * src/device/coopmat_intrinsics.jl:16-19; same contract as the f16 form). */
int lava_hip_gemm_bf16_f32(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                           int64_t ldb, int64_t ldc, uint32_t layout, void* stream);
/* int8 x int8 -> int32, all operands signed (src/compiler/spirv/coopmat.jl:115-151),
 * exact with two's-complement wrap of the 32-bit accumulator. */
int lava_hip_gemm_i8_i32(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                         int64_t ldb, int64_t ldc, uint32_t layout, void* stream);

/* uint8 x uint8 -> uint32, all operands unsigned (src/compiler/spirv/coopmat.jl:115-151 emits no
 * signed-component bits for UInt8 coopmats; test/spirv/test_coopmat_int8.jl:71-98), exact with
 * the 32-bit accumulator's wrap; C holds uint32.  The MFMA is signed only: the tile, mid-size
 * and small-product kernels multiply the bytes flipped by 128 (u - 128) and add 128 (row sum +
 * column sum) + 16384 K back after their last k-step.  The kernel choice is the signed one's
 * (tile kernel, 128 x 128 mid-size kernel, small-product kernel with K split through the
 * per-stream workspace, in their unsigned forms); shapes no MFMA kernel takes (a K-contiguous K or
 * an M/N-contiguous M/N not a multiple of 16, 16-byte misaligned operands or leading dimensions)
 * run on a one-thread-per-element kernel.  Same layouts and leading-dimension rules as above. */
int lava_hip_gemm_u8_u32(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                         int64_t ldb, int64_t ldc, uint32_t layout, void* stream);

/* The coopmat2 (tensor-addressed, workgroup-scope) GEMM: C = fp16(A B), fp32 accumulate.
 * A (M x K) and B (K x N) fp16 row-major, zero-clamped so that any M, N, K works unpadded;
 * C row-major M x N (ldc >= N) or, with LAVA_HIP_CM2_TRANSPOSE_C, C^T stored row-major
 * N x M (ldc >= M) through the transposing view.  Extents and leading dimensions < 2^31.
 * Default: the 256 x 256 tile kernel (buffer-resource loads that read zero past the
 * extent); LAVA_HIP_CM2_VOCABULARY: the shader's own form in the tensor vocabulary
 * (128 x 128 blocks, K steps of 64, tensor_load / tensor_store per fragment).
 * Replaces `gemm_cm2!` / test/glsl/coopmat2_gemm_regs.comp:37-84 (push block
 * {pa, pb, pc, M, N, K}), with the view store of tensor_intrinsics.jl:371-402. */
#define LAVA_HIP_CM2_TRANSPOSE_C 1u
#define LAVA_HIP_CM2_VOCABULARY 2u
int lava_hip_gemm_cm2_f16(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda,
                          int64_t ldb, int64_t ldc, uint32_t flags, void* stream);

/* ---- fused GEMM epilogue: activations (elementwise epilogues that Lava writes with
 * coopmat_length / getcomp / setcomp, src/device/coopmat_intrinsics.jl:322-400) ---- */
#define LAVA_HIP_ACT_NONE 0
#define LAVA_HIP_ACT_RELU 1
#define LAVA_HIP_ACT_GELU_TANH 2 /* 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) */
#define LAVA_HIP_ACT_GELU_ERF 3  /* 0.5 x (1 + erf(x / sqrt(2))) */

/* GEMM with the epilogue family fused into the store:
 *   D = act(A B + (bias + residual)), narrowed RNE to D's type.
 * The accumulator init is Lava's `accinit`: a stride-0 accumulator load of the bias (one
 * fp32 value per row m of D) plus the residual (fp32, M x N, laid out like D with leading
 * dimension ldr), summed with coopmat_add (src/device/coopmat_intrinsics.jl:435-464;
 * src/compiler/spirv/coopmat.jl:870-885); `act` is the getcomp/setcomp epilogue; the
 * fp16 / bf16 output is coopmat_convert of the fp32 accumulator, RNE
 * (src/compiler/spirv/coopmat.jl:163-182, 783-824).
 * ab_dtype: LAVA_HIP_F16 or LAVA_HIP_BF16 (A and B); d_dtype: LAVA_HIP_F32, LAVA_HIP_F16 or
 * LAVA_HIP_BF16.  bias and residual may each be NULL (ldr is then unused); layout as for the
 * plain GEMM, bit 2 giving D's and the residual's layout.  The plain entry points are this
 * call with no bias, no residual, LAVA_HIP_ACT_NONE and an fp32 D. */
int lava_hip_gemm_ex(int ab_dtype, int d_dtype, const void* A, const void* B, void* D, int64_t M, int64_t N,
                     int64_t K, int64_t lda, int64_t ldb, int64_t ldd, uint32_t layout, const float* bias,
                     const float* residual, int64_t ldr, int act, void* stream);

/* The 16x16x16 subgroup-tile GEMM written directly in the vocabulary, one
 * wavefront per 16x16 tile of C, loading straight from global as
 * docs/src/device.md:81-88 does (fp16 in, fp32 out).  M, N, K multiples of 16. */
int lava_hip_coopmat_gemm_f16_tiles(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K,
                                    int64_t lda, int64_t ldb, int64_t ldc, uint32_t layout, void* stream);

/* W8A16 (coopmat2 per-element dequant callback, src/device/coopmat_intrinsics.jl:535-628
 * with the scale pointer in `extras`, :569-572):
 *   Y (M x N, fp32) = (X (M x K, fp16) * float(W (K x N, int8))) .* s[col] (fp16).
 * layout: bit0 X row-major, bit1 W row-major, bit2 Y row-major.  Two weight-streaming
 * kernels, every call one launch:
 *  - W column-major (K contiguous per output column), X and Y either way: any N, K a
 *    multiple of 16, 16-byte aligned W with a leading dimension a multiple of 16.  Whole
 *    columns per workgroup, for 1, 2 or 4 16-row blocks of X (M up to 16, 32, or more): W is
 *    streamed once per 64 rows at most.  X is read in place when row-major (16-byte aligned, ldx a multiple of 8),
 *    or column-major with M a multiple of 8 (or M == 1 with ldx == 1); any other column-major X
 *    is first copied row-major into the workspace (M x K fp16).
 *  - W row-major, X and Y either way: K a multiple of 32, N of 8, 8-byte aligned W with ldw
 *    a multiple of 8 (a row-major X 16-byte aligned with ldx a multiple of 8).  Narrower N
 *    splits K across workgroups, whose last-arriving workgroup per column block adds the
 *    partial blocks from the workspace.
 * The workspace (split-K partials, or the copy of X) is owned by the library, one per
 * (device, stream): a call that grows it allocates (hipMalloc).  A call on a stream that is
 * capturing a graph never allocates: it plans within the workspace the stream already has
 * (fewer K splits, or the generic kernel instead of the copy of X; same results to rounding
 * of the split sums) -- make one call of the largest shape outside capture first to capture
 * the same plan.  A graph captured with a workspace holds its address: the buffer is then kept
 * until the process ends, and replaying the graph while calls on its capture stream run
 * races on it (serialise them).  Calls on one stream from several threads are serialised
 * around the workspace; lava_hip_stream_destroy and lava_hip_release_workspaces free it.
 * Any other layout or shape runs on a generic kernel.  Results are deterministic (fixed
 * summation order). */
int lava_hip_gemm_w8a16(const void* X, const void* W, const void* scale, void* Y, int64_t M, int64_t N, int64_t K,
                        int64_t ldx, int64_t ldw, int64_t ldy, uint32_t layout, void* stream);

/* lava_hip_gemm_w8a16 without any allocation: the same kernels and results (bit for bit),
 * with the workspace (split-K arrival counters and partial blocks, or the row-major copy of a
 * column-major X) in a fixed per-GPU device array of LAVA_HIP_W8A16_NOALLOC_SCRATCH_BYTES
 * instead of a library-allocated one -- except that a column-major X whose copy would not fit
 * (M not a multiple of 8 and M x K above 1 M elements) runs on the generic kernel.  No
 * counterpart in the reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No call makes a hipMalloc,
 * hipFree or other allocating call; a shape whose plan needs more scratch than the array holds
 * is refused with LAVA_HIP_ERR_INVALID_ARG (no plan of the split rule does).  Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (two streams, two threads) race
 * and must be serialised by the caller. */
#define LAVA_HIP_W8A16_NOALLOC_SCRATCH_BYTES (((size_t)2 << 20) + 4096)
int lava_hip_gemm_w8a16_noalloc(const void* X, const void* W, const void* scale, void* Y, int64_t M, int64_t N,
                                int64_t K, int64_t ldx, int64_t ldw, int64_t ldy, uint32_t layout, void* stream);

/* Flash-attention forward, fp16 Q/K/V/O, fp32 running max and sum:
 *   O = softmax(Q K^T * scale + mask) V  per (head, batch),
 * the `attn_flash_rows!` / flash_attn_cm2 form (src/vocabulary/coopmat.jl:158;
 * src/device/coopmat_intrinsics.jl:638-720).  Tensors are (E, L, H, B) = (D, S, H, B):
 * element (e, l, h, b) at e*st[0] + l*st[1] + h*st[2] + b*st[3]
 * (src/device/tensor_intrinsics.jl:279-281).  causal != 0 masks key > query.
 * Q, K, V share `strides`; O uses `ostrides` (NULL = same as strides).  MFMA kernels take
 * D <= 128 (a multiple of 8), and 128 < D <= 256 (a multiple of 8) with scale > 0 (two
 * launches, one per 128-column half of V and O), when Q, K and V are 16-byte aligned with
 * strides[1..3] multiples of 8 and O is 8-byte aligned with ostrides[1..3] multiples of 4; any
 * other D (<= 256) or layout runs on a generic kernel (one thread per query). */
int lava_hip_flash_attn_fwd_f16(const void* Q, const void* K, const void* V, void* O, int64_t B, int64_t H, int64_t S,
                                int64_t D, const int64_t* strides, const int64_t* ostrides, float scale, int causal,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LAVA_HIP_H */
