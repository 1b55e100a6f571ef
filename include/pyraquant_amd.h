/*
 * pyraquant_amd.h -- C ABI of libpqint8.so, the MI355X (gfx950) INT8 deployment hot path.
 *
 * The library replaces the GPU kernels behind PyraQuant's `Int8Linear` executor
 * (reference: deploy/int8_exec.py, deploy/run_sdxl_latency.py). Every entry point takes raw device
 * pointers, element strides and a HIP stream; no entry point allocates, frees or clears device memory with a
 * runtime call (hipMalloc, hipFree, hipMemset*), and none synchronises the stream. All calls are asynchronous
 * on `stream` (pass the caller's current stream; torch: torch.cuda.current_stream().cuda_stream). Memory the
 * kernels use beyond their inputs and outputs is the caller's: the GEMMs' optional scheduling buffer (`sched`)
 * and pq_int8_linear's workspace. The one exception is pq_int8_linear_noalloc's staging, a 64 MiB static device
 * array that the HIP runtime maps on every GPU the library's code object is loaded on, whether or not that
 * entry point is ever called. The C API keeps no other mutable global state apart from the thread-local error
 * text, so every entry point other than pq_int8_linear_noalloc may be called from several host threads.
 *
 * Return value of every int-returning entry point: PQ_OK (0) or a negative PQ_E* code; the text of the
 * last error on the calling thread is available from pq_last_error().
 *
 * Layout contract (all matrices row-major, last dimension contiguous, strides in elements):
 *   activations x   [M, K]  bf16 or fp16, row stride ldx >= K      (reference: deploy/int8_exec.py:216-230)
 *   codes       q   [M, K]  int8, contiguous (row stride K)        (reference: deploy/int8_exec.py:225)
 *   row scales  s   [M]     fp32
 *   weights     w   [N, K]  int8, row stride ldw (K-contiguous, "TN") (reference: deploy/int8_exec.py:150, 358)
 *   per-channel scales s_w [N] fp32                                 (reference: deploy/int8_exec.py:356, 359)
 *   group-32 scales    s_w [K/32, N] fp32 (group-major: one row of N scales per 32-wide K group)
 *   low-rank down  l1t [R, K] bf16/fp16  = transpose of the reference's lr_A [K, R] (deploy/int8_exec.py:376)
 *   low-rank up    l2t [N, R] bf16/fp16  = transpose of the reference's lr_B [R, N] (deploy/int8_exec.py:377)
 *   low-rank mid   t   [M, R] bf16/fp16, row stride ldt             (reference: deploy/int8_exec.py:390)
 *   output      c   [rows, N] bf16/fp16, row stride ldc
 *
 * Packed K64 layout (pq_pack_k64, pq_quant_rows_packed, pq_int8_gemm_packed) of an int8 matrix X [R, K], K % 64 == 0:
 * KT = K / 64 and RB = ceil(R / 16) blocks of 1024 bytes per row block; block (rb, kt) sits at byte offset
 * (rb * KT + kt) * 1024 and holds rows 16 rb .. 16 rb + 15, bytes 64 kt .. 64 kt + 63 of each. Row r' (= r % 16)
 * occupies bytes [64 r', 64 r' + 64) of the block and stores its 16-byte chunk c (bytes 64 kt + 16 c ..) at slot
 * c ^ swz(r'), swz(r') = ((r' >> 2) & 1) | ((((r' >> 1) ^ (r' >> 3)) & 1) << 1). Size RB * KT * 1024 bytes; rows
 * past R in the last block are zero. A block is the exact LDS image the GEMM's MFMA operand reads expect, so the
 * GEMM moves it with one 1 KB LDS-DMA per wave and every request is a whole 128-byte line.
 */
#ifndef PYRAQUANT_AMD_H
#define PYRAQUANT_AMD_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PQ_ABI_VERSION 3

/* status codes */
#define PQ_OK 0
#define PQ_EINVAL (-1)  /* null pointer or invalid argument              -> Python AssertionError */
#define PQ_ESHAPE (-2)  /* unsupported shape (e.g. K % 64 != 0)           -> Python AssertionError */
#define PQ_EALIGN (-3)  /* pointer / stride alignment not supported       -> Python AssertionError */
#define PQ_EDTYPE (-4)  /* unsupported dtype code                         -> Python ValueError     */
#define PQ_ELAUNCH (-5) /* HIP runtime error at launch                    -> Python RuntimeError   */

/* element type codes of the 16-bit floating operands (and, for pq_int8_gemm_packed's output, raw int32) */
#define PQ_BF16 0
#define PQ_F16 1
#define PQ_I32 2

/* flag OR'ed into pq_int8_gemm_packed's out_dtype: accumulate into c instead of overwriting it,
 * c[o, n] = round(c[o, n] + round(y)) (two 16-bit roundings, as torch adds two 16-bit tensors) */
#define PQ_ACCUMULATE 0x100

/* Version of this ABI (PQ_ABI_VERSION). No reference counterpart. */
int pq_abi_version(void);

/* Text of the last error raised on the calling thread ("" if none). No reference counterpart: the
 * reference reports errors as Python exceptions (deploy/int8_exec.py:67-68, 206, 221, 235). */
const char* pq_last_error(void);

/*
 * Per-token activation quantizer, with an optional fused row gather.
 * Replaces `quant_rows` / `_quant_rows_kernel` (deploy/int8_exec.py:78-101, 216-230) and the SDXL direct
 * launch `fast_quant_rows` (deploy/run_sdxl_latency.py:159-170).
 *
 * For output row m (0 <= m < M) the source row is r = row_idx ? row_idx[m] : m, and
 *   a    = max(max_k |x[r, k]|, 1e-8f)
 *   s[m] = a / 127.0f                                    (IEEE fp32 division, round to nearest even)
 *   q[m, k] = clamp(rint(x[r, k] / s[m]), -127, 127)     (IEEE fp32 division, rint = half to even)
 * which is the reference's torch restatement (deploy/int8_exec.py:508-509). q is [M, K] contiguous.
 * x has x_rows rows (x_rows >= M without row_idx). A row_idx entry outside [0, x_rows) reads as a row of zeros
 * (codes 0, s = fl(1e-8) / 127) instead of memory past x; torch's index ops would raise there.
 * Inputs must be finite. Any K >= 1 and ldx >= K are accepted; 16-byte aligned x with ldx % 8 == 0 and
 * K % 8 == 0 takes the vectorised kernel, anything else a per-element kernel with the same results.
 */
int pq_quant_rows(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                  const int32_t* row_idx, int8_t* q, float* s, hipStream_t stream);

/*
 * Weight round-to-nearest quantization (one-off, at module conversion). w is [N, K] fp32 with row stride ldw.
 *   group == 0 : s[n]       = max(max_k |w[n, k]|, 1e-8f) / 127           (IEEE fp32 division)
 *   group == g : s[n, j]    = max(max_{k in [jg, jg+g)} |w[n, k]|, 1e-8f) / 127   (g divides K)
 *   q[n, k] = clamp(rint(w[n, k] / s), -127, 127), q [N, K] contiguous, s [N] or [N, K / g] contiguous.
 * Replaces the weight RTN of `Int8Linear.__init__` (deploy/int8_exec.py:352-357) and, for group > 0, the codes
 * and scales of `qdq_weight(w, 8, group)` (pyraquant/quantizers_weight.py:96-109).
 */
int pq_quant_weight(const float* w, int64_t N, int64_t K, int64_t ldw, int64_t group, int8_t* q, float* s,
                    hipStream_t stream);

/*
 * Low-rank down-projection t = x[rows] @ lr_A, fp32 accumulation, rounded to the 16-bit type of x.
 * Replaces `t = x2.to(self.lr_A.dtype) @ self.lr_A` (deploy/int8_exec.py:390; also :403).
 * x is [x_rows, ldx] (the rows row_idx may name; without row_idx x_rows >= M). x and l1t must have the same dtype.
 * l1t is lr_A transposed ([R, K], K-contiguous). R in {32, 64, 96, 128}, K % 8 == 0, 16-byte aligned x / l1t / t,
 * ldx % 8 == 0, ldt % 8 == 0. row_idx as in pq_quant_rows (the routed gather; entries outside [0, x_rows) read as zero
 * rows), or NULL. K % 64 == 0 and R <= 64 take
 * the LDS-DMA kernel (x streamed once in whole 128-byte row segments); other shapes a per-row-fragment kernel.
 */
int pq_lowrank_down(const void* x, int32_t dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                    const int32_t* row_idx, const void* l1t, int64_t R, void* t, int64_t ldt,
                    hipStream_t stream);

/*
 * Fused INT8 GEMM + dequant epilogue, one kernel. For 0 <= m < M, 0 <= n < N:
 *   group == 0 : y = (float)(sum_k a[m,k] * w[n,k]) * (s_row[m] * s_w[n])
 *   group == 32: y = s_row[m] * sum_g s_w[g, n] * (float)(sum_{k in g} a[m,k] * w[n,k])
 *   if t   : y += sum_r t[m, r] * l2t[n, r]     (fp32 accumulation of the 16-bit operands)
 *   if bias: y += bias[n]
 *   c[o, n] = round_to_out_dtype(y), o = out_row_idx ? out_row_idx[m] : m (routed scatter)
 * The int32 accumulator never leaves registers. Rows of c not named by out_row_idx are not written,
 * so they keep whatever the caller left there (the routed executor's cached canvas). With out_row_idx, c has
 * c_rows rows, and a row whose index lies outside [0, c_rows) is not written (torch's index ops would raise); without
 * it c has M rows and c_rows is ignored.
 * Replaces `int8_gemm_fused` / `_int8_gemm_fused_kernel_impl` (deploy/int8_exec.py:144-183, 202-212),
 * `int8_gemm_lr` / `_int8_gemm_lr_impl` (deploy/int8_exec.py:272-314, 327-336; epilogue order
 * :303-309), the SDXL narrow-N variant (deploy/run_sdxl_latency.py:131-140, 173-195). The group-32
 * form and the scatter have no reference kernel (weight semantics: pyraquant/quantizers_weight.py:96-109).
 * Requirements: K % 64 == 0, N % 64 == 0, M >= 1; a, w 16-byte aligned with lda, ldw % 16 == 0;
 * c 8-byte aligned with ldc % 4 == 0 and ldc < 2^31; t, l2t 16-byte aligned with ldt % 8 == 0, ldt <= 2^22,
 * R in {16, 32, 64}; group 32 needs N * K < 2^33 (its scales are read at 32-bit buffer offsets);
 * lr_dtype and out_dtype are PQ_BF16 or PQ_F16; out_row_idx entries unique (two rows naming one row of c race).
 * sched: NULL, or a scheduling buffer of 9 int32 (36 bytes, 4-byte aligned) on the stream's device that the
 * caller owns. Large products (rank 0-32, no accumulate, more 256 x 256 blocks than CUs) run one persistent
 * workgroup per CU. With a buffer, the workgroups claim blocks from per-XCD counters in it, so the faster XCDs take
 * the slower ones' last blocks; without one, each takes a fixed share. The buffer must hold zeros when the launch
 * starts (e.g. torch.zeros once), and every launch leaves it zeroed, so launches ordered on one stream may share it
 * and launches that may overlap (other streams, a graph replayed beside eager work) must not. Smaller products
 * ignore it. The results do not depend on the schedule.
 */
int pq_int8_gemm(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw,
                 const float* s_row, const float* s_w, int64_t group, const float* bias,
                 const void* t, int64_t ldt, const void* l2t, int64_t R, int32_t lr_dtype,
                 void* c, int64_t ldc, int32_t out_dtype, const int32_t* out_row_idx, int64_t c_rows,
                 int64_t M, int64_t N, int64_t K, int32_t* sched, hipStream_t stream);

/*
 * int32 accumulator only: c[m, n] = sum_k a[m, k] * w[n, k] (exact). The bit-exact check of the
 * MFMA contraction; the same kernel body as pq_int8_gemm. Replaces `torch._int_mm(xq, w_int8.t())`
 * (deploy/int8_exec.py:259). Requirements as pq_int8_gemm, c 16-byte aligned.
 */
int pq_int8_gemm_i32(const int8_t* a, int64_t lda, const int8_t* w, int64_t ldw, int32_t* c,
                     int64_t ldc, int64_t M, int64_t N, int64_t K, hipStream_t stream);

/*
 * Per-token quantizer (packed K64 codes, as pq_quant_rows_packed) and the rank-R low-rank down-projection
 * t = x[rows] @ L1 (as pq_lowrank_down) from one pass over x: the two steps of Int8Linear.forward that read x,
 * `t = x2.to(lr_A.dtype) @ lr_A` and `quant_rows(x2)` (deploy/int8_exec.py:390-391). qp / s are bit-identical to
 * pq_quant_rows_packed; t is the fp32-accumulated product rounded to the 16-bit type, as pq_lowrank_down (the
 * accumulation order differs, so the last bit of t may differ from it). x is read from HBM once when R == 32, rows
 * are 16-byte aligned (ldx % 8 == 0) and K is one of 1024, 1280, 2048, 2560, 3072 (rows staged through LDS; every x
 * byte offset must fit 30 bits) or 4096, 6144, 8192, 10240, 12288, 15360 (rows held in registers); other shapes run
 * the two kernels. l1t [R, K] contiguous, same dtype as x; t [M, R] with row stride ldt.
 * l1f: NULL, or the same matrix in the one-pass kernel's fragment order (pq_pack_lowrank_l1t, 16-byte aligned),
 * which that kernel then reads instead of l1t (contiguous 1 KB register loads: 15.8 -> 12.8 us at M = 4096,
 * K = 3072); results are identical either way, and l1t is still required (the other paths read it).
 */
int pq_quant_rows_lowrank(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                          const int32_t* row_idx, const void* l1t, const void* l1f, int64_t R, int8_t* qp, float* s,
                          void* t, int64_t ldt, hipStream_t stream);

/*
 * Write l1t [R, K] (bf16/fp16, contiguous, 16-byte aligned) in the fragment order pq_quant_rows_lowrank's one-pass
 * kernel loads from its l1f argument: l1f receives R * K 16-bit values (16-byte aligned). Defined for R == 32 and
 * K in {1024, 1280, 2048, 2560, 3072} (the one-pass shapes); PQ_ESHAPE otherwise, and callers then pass l1f = NULL.
 * One-off at weight conversion, like pq_pack_k64. No reference counterpart (the reference multiplies by lr_A
 * [K, R] with torch, deploy/int8_exec.py:390).
 */
int pq_pack_lowrank_l1t(const void* l1t, int32_t dtype, int64_t R, int64_t K, void* l1f, hipStream_t stream);

/*
 * Fused INT8 GEMM over packed K64 operands (ap: activation codes [M, K], wp: weights [N, K], both in the packed
 * K64 layout). Same math, epilogue, scatter and requirements as pq_int8_gemm (group 0: s_w [N]; group 32:
 * s_w [K/32, N] group-major); with out_dtype == PQ_I32, c receives the raw int32 accumulator (s_row, s_w, group,
 * bias, t, l2t, out_row_idx ignored; c 16-byte aligned, ldc % 4 == 0). With out_dtype | PQ_ACCUMULATE (16-bit
 * output, group 0), each output element is added to what c holds: c = round(c + round(y)), so a Linear split along
 * its input accumulates its second half into the first half's output in the same pass that writes it
 * (`SplitInLinear.forward`'s `L0(x0) + L1(x1)`, pyraquant/external_quant.py:191-192). This is the layer path of Int8Linear: the quantizer writes ap directly
 * (pq_quant_rows_packed) and the weights are packed once at conversion (pq_pack_k64). sched as pq_int8_gemm
 * describes (ignored with PQ_I32 or PQ_ACCUMULATE).
 * Replaces `int8_gemm_fused` / `int8_gemm_lr` (deploy/int8_exec.py:202-212, 327-336) as called from
 * `Int8Linear.forward` (deploy/int8_exec.py:382-393).
 */
int pq_int8_gemm_packed(const int8_t* ap, const int8_t* wp, const float* s_row, const float* s_w, int64_t group,
                        const float* bias, const void* t, int64_t ldt, const void* l2t, int64_t R, int32_t lr_dtype,
                        void* c, int64_t ldc, int32_t out_dtype, const int32_t* out_row_idx, int64_t c_rows,
                        int64_t M, int64_t N, int64_t K, int32_t* sched, hipStream_t stream);

/*
 * Bytes of workspace pq_int8_linear needs for M rows, K inputs and R columns of t (R = 0: no low-rank branch):
 * the packed codes, the row scales, t and the GEMM's 36-byte scheduling buffer, each slice starting on a 256-byte
 * boundary. -1 for a bad argument.
 * No reference counterpart (the reference allocates the three tensors per call with torch.empty,
 * deploy/int8_exec.py:225-226, 390).
 */
int64_t pq_int8_linear_workspace_size(int64_t M, int64_t K, int64_t R);

/*
 * A whole Int8Linear layer in one call: y = Linear(x) as pq_quant_rows_lowrank (R > 0) or pq_quant_rows_packed
 * (R == 0) followed by pq_int8_gemm_packed, with the codes, row scales and t staged in `workspace` (at least
 * pq_int8_linear_workspace_size(M, K, R) bytes, 256-byte aligned; its contents on entry do not matter, and it is
 * in use until the GEMM has run on `stream`). x [M, K] bf16/fp16 (row stride ldx); w_packed the packed K64
 * weights [N, K]; s_w [N] (group 0) or [K/32, N] (group 32); bias [N] fp32 or NULL; l1t [R, K] and l2t [N, Re] in
 * x's dtype (R a multiple of 32 up to 128, Re in {16, 32, 64} and Re <= R: the first Re columns of t enter the
 * epilogue), or NULL with R = Re = 0; l1f NULL or l1t in fragment order (as pq_quant_rows_lowrank); y [M, N] in
 * x's dtype with row stride ldy. Same results as the two calls. The workspace also holds the GEMM's scheduling
 * buffer (pq_int8_gemm's sched), which the quantizer kernel zeroes, so a large layer claims its blocks even when
 * replayed from a graph; calls that may overlap need workspaces of their own.
 * Replaces the body of `Int8Linear.forward` (deploy/int8_exec.py:382-393): one C call per layer.
 */
int pq_int8_linear(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* w_packed,
                   const float* s_w, int64_t group, const float* bias, const void* l1t, const void* l1f, int64_t R,
                   const void* l2t, int64_t Re, void* y, int64_t ldy, int64_t N, void* workspace, int64_t ws_bytes,
                   hipStream_t stream);

/*
 * pq_int8_linear without a workspace argument. No counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The workspace (codes, scales, t and the scheduling buffer) lives in a static device array of the library,
 * pq_int8_linear_noalloc_max_bytes() bytes (64 MiB). The runtime maps that array on every GPU the library's code
 * object is loaded on, whether or not this entry point is called, and holds it until the process ends. A layer
 * whose pq_int8_linear_workspace_size(M, K, R) exceeds it is refused with PQ_ESHAPE before any work (FLUX's
 * 1K-stage and SDXL's layers fit; FLUX's 4K stage does not). Nothing is allocated or freed per call. `stream` must
 * belong to the current device. Every call on a GPU uses that GPU's one array: calls that overlap on one GPU
 * (other streams, other threads) race, so serialise them. The other arguments and the result are those of
 * pq_int8_linear.
 */
int pq_int8_linear_noalloc(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, const int8_t* w_packed,
                           const float* s_w, int64_t group, const float* bias, const void* l1t, const void* l1f,
                           int64_t R, const void* l2t, int64_t Re, void* y, int64_t ldy, int64_t N,
                           hipStream_t stream);

/* Bytes of the device array behind pq_int8_linear_noalloc (its largest staging). No reference counterpart. */
int64_t pq_int8_linear_noalloc_max_bytes(void);

/*
 * Repack a row-major int8 matrix src [R, K] (row stride lds, K % 64 == 0) into the packed K64 layout at dst
 * (ceil(R / 16) * 16 * K bytes, 16-byte aligned); padding rows are written as zeros. One-off at weight
 * conversion. No reference counterpart (the reference's Triton GEMM reads W_int8 row-major,
 * deploy/int8_exec.py:165-166).
 */
int pq_pack_k64(const int8_t* src, int64_t R, int64_t K, int64_t lds, int8_t* dst, hipStream_t stream);

/*
 * Per-token quantizer writing the codes in the packed K64 layout (qp: ceil(M / 16) * 16 * K bytes, 16-byte
 * aligned; padding rows zero) instead of row-major; s and every other argument as pq_quant_rows. K % 64 == 0.
 * Replaces `quant_rows` (deploy/int8_exec.py:216-230) on the Int8Linear forward path (:391).
 */
int pq_quant_rows_packed(const void* x, int32_t x_dtype, int64_t M, int64_t K, int64_t ldx, int64_t x_rows,
                         const int32_t* row_idx, int8_t* qp, float* s, hipStream_t stream);

/*
 * Dequant epilogue over a materialised int32 accumulator:
 *   c[m, n] = round_to_out_dtype((float)acc[m, n] * (s_row[m] * s_col[n]) (+ bias[n])).
 * Replaces `dequant_epilogue` / `_dequant_epilogue_kernel` (deploy/int8_exec.py:104-127, 233-243).
 * acc is [M, N] contiguous int32.
 */
int pq_dequant_epilogue(const int32_t* acc, const float* s_row, const float* s_col, const float* bias,
                        void* c, int64_t ldc, int32_t out_dtype, int64_t M, int64_t N,
                        hipStream_t stream);

/* ---- routed executor: geometry and fusion on the device ------------------------------------------------------
 * The leaf mask `sel` is uint8 [Lh, Lw] on the device (nonzero = selected; the reference thresholds its mask at
 * 0.5, flux/run_flux.py:343). Token (y, x) of the H x W packed-token grid is row y * W + x
 * (flux/routing.py:105-115). Counts are written to device memory, so no call waits for the host.
 */

/*
 * Linear-level gather list: the sorted, unique token rows covered by the union of the selected leaves
 * (leaf_tokens x leaf_tokens tokens each), each dilated by `halo` tokens and clamped to the grid
 * (flux/routing.py:235-244). rows holds up to H * W entries; *count receives their number. Requires
 * Lh * leaf_tokens <= H, Lw * leaf_tokens <= W, Lw <= 64, Lh <= 1024 and Lh * Lw <= 32768. The reference builds its row sets on the host
 * from sel.cpu() (flux/run_flux.py:343-355, flux/routing.py:253-315); this list is the union of those patches.
 */
int pq_route_union_rows(const uint8_t* sel, int64_t Lh, int64_t Lw, int64_t leaf_tokens, int64_t halo, int64_t H,
                        int64_t W, int32_t* rows, int32_t* count, hipStream_t stream);

/*
 * Patch extraction geometry of the routed executor:
 *   boxes  : row-wise runs of selected leaves, leaf_latent latent cells each (flux/run_flux.py:340-355);
 *   cores  : latent box -> packed-token box with the 2x2 packing phase packing_offset (flux/routing.py:202-232);
 *            repeated cores are dropped (:276-278);
 *   patches: core dilated by `halo` tokens, clamped (:235-244), grouped by shape in ascending (h, w) order, box
 *            order inside a shape (:298-315).
 * table [patches, 12] int32, per patch in extraction order: halo box oy0, oy1, ox0, ox1; core box cy0, cy1, cx0,
 * cx1; first row of the patch in `rows`; source box index; bucket (shape rank); 0. Room for Lh * ceil(Lw / 2)
 * patches. counts[4] int32: patches, rows, buckets, error bits (1 = more than max_rows rows; those patches' rows
 * are not written). rows [max_rows] int32: every patch's token rows, row-major inside the patch, patches in
 * order -- the order in which build_patch_buckets stacks hidden_states (:286-296). max_rows = 0 computes the
 * table only. Requires leaf_latent even, Lh <= 1024, Lh * Lw <= 32768, Lh * ceil(Lw / 2) <= 2048, H, W <= 32767
 * and the leaf grid inside the token grid.
 */
int pq_route_patches(const uint8_t* sel, int64_t Lh, int64_t Lw, int64_t leaf_latent, int64_t halo, int64_t H,
                     int64_t W, int64_t packing_offset, int32_t* table, int32_t* counts, int32_t* rows,
                     int64_t max_rows, hipStream_t stream);

/*
 * Row gather with a device-side count: dst row r = src row rows[r] for r < min(*count, n_max), row_bytes bytes per
 * row (multiple of 4), strides in bytes. The patch extraction of hidden_states / img_ids in build_patch_buckets
 * (flux/routing.py:286-296), without the host learning the row count.
 */
int pq_gather_rows(const void* src, int64_t ld_src_bytes, const int32_t* rows, const int32_t* count, int64_t n_max,
                   int64_t row_bytes, void* dst, int64_t ld_dst_bytes, hipStream_t stream);

/*
 * Feathered fusion of the patch predictions into the background (fuse_patch_predictions, flux/routing.py:328-379,
 * with halo_feather_mask :34-75, min_alpha 0):
 *   per patch covering a token, in table order: beta = (fusion_beta * mask).clamp(0, 1);
 *   local += beta * out; beta_acc += beta  (every product and sum rounded to the 16-bit type, as torch does);
 *   result = (1 - clamp(beta_acc, 0, 1)) * bg + clamp(beta_acc, 0, 1) * where(beta_acc > 0, local / beta_acc, 0).
 * mask = min(y ramp, x ramp) over the halo, 1 over the core. ramp holds, for every ramp length m = 1 .. halo
 * (the halo of the route table, at most 64), the
 * rising ramp r(linspace(0, 1, m)) and the falling ramp r(linspace(1, 0, m)) interleaved:
 * ramp[2 (m (m - 1) / 2 + u)] and ramp[2 (m (m - 1) / 2 + u) + 1] (fp32; the caller evaluates the reference's
 * _smooth_ramp, flux/routing.py:21-31, once per halo and mode). background / out [H * W, C] (row strides ldb /
 * ldo), patch_out [rows, C] (row stride ldp) holds the patch predictions in the order of `rows` from
 * pq_route_patches; table / counts from pq_route_patches. C % 8 == 0, 16-byte aligned rows, dtype bf16 or fp16.
 */
int pq_fuse_patches(const void* background, int64_t ldb, const void* patch_out, int64_t ldp, const int32_t* table,
                    const int32_t* counts, const float* ramp, int64_t halo, float fusion_beta, int64_t H, int64_t W,
                    int64_t C, int32_t dtype, void* out, int64_t ldo, hipStream_t stream);

/* ---- weight-side conversion ------------------------------------------------------------------------------ */

/*
 * Smoothing / shift fold of an SVDQuant package Linear, one pass over its 16-bit weight w [N, K] (row stride ldw):
 *   Wf = (float)w / smooth                          (smooth: NULL, one fp32 scalar (n_smooth 1) or [K] fp32)
 *   w_out[n, k] = Wf[n, k] rounded to dtype          (w_out may be w: in place; row stride ldo)
 *   add[n] = sum_k Wf[n, k] * shift[k]  ([K] shift)  or  (sum_k Wf[n, k]) * shift[0]  (scalar shift)
 *   bias_out[n] = round(bias_in[n] + round(add[n])) (bias_in NULL: round(add[n])), 16-bit dtype, may alias bias_in.
 * Without shift bias_out may be NULL (the bias is unchanged). The shift sum is fp32 in an order of this kernel's
 * own, so it agrees with torch's matmul to rounding. Replaces `_fold_one` (deploy/run_flux_latency.py:210-239) on
 * the Int8Linear path, which then quantizes the folded weight (pq_quant_weight).
 */
int pq_fold_weight(const void* w, int32_t dtype, int64_t N, int64_t K, int64_t ldw, const float* smooth,
                   int64_t n_smooth, const float* shift, int64_t n_shift, const void* bias_in, void* w_out,
                   int64_t ldo, void* bias_out, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PYRAQUANT_AMD_H */
