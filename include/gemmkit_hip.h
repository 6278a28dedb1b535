/*
 * gemmkit_hip.h -- C ABI of the MI355X (gfx950) GEMM engine.
 *
 * The entry points mirror gemmkit's public Rust API one for one (the citations
 * are gemmkit/src/... file:line of the function each one replaces), so a
 * `-sys` binding can sit behind the same Rust signatures:
 *   - the checked tier takes strided views with their slice lengths
 *     (MatRef/MatMut, src/api.rs:92-180) and reproduces the reference's
 *     validation, returning an error code where the reference panics;
 *   - the `_unchecked` tier takes raw pointers and element strides, exactly the
 *     reference's `*_unchecked_with` argument lists (negative strides allowed);
 *   - every entry takes a `gk_workspace*` first: NULL means the library's own
 *     per-thread workspace (the reference's thread-local pool,
 *     src/workspace.rs:225-246), non-NULL is the `_with(&mut Workspace, ..)` twin.
 *
 * All matrix pointers are DEVICE pointers (HBM).  By default every call is
 * synchronous like the reference (C is complete on return); gk_set_synchronous(0)
 * turns calls into stream-ordered launches on the stream set by gk_set_stream.
 *
 * Return value: GK_OK (0) or a negative gk_status; gk_last_error() then holds
 * the message, worded as the reference's panic message ("gemmkit: ...").
 * Element strides are in elements, as in the reference.
 */
#ifndef GEMMKIT_HIP_H
#define GEMMKIT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status */

typedef enum gk_status {
    GK_OK = 0,
    GK_ERR_SHAPE = -1,       /* dimension mismatch (reference: assert_eq! panics)      */
    GK_ERR_VIEW = -2,        /* view out of its slice, negative stride, bad batch stride */
    GK_ERR_ALIAS = -3,       /* C aliases itself / A / B / bias / scales              */
    GK_ERR_ARG = -4,         /* scale or zero-point out of range, bad enum value      */
    GK_ERR_LAYOUT = -5,      /* prepacked-B call with a row-major-ish C               */
    GK_ERR_OVERFLOW = -6,    /* a size computation overflows                          */
    GK_ERR_DEVICE = -7,      /* HIP runtime failure or no device                      */
    GK_ERR_NOMEM = -8        /* device allocation failed                              */
} gk_status;

/* Message of the last failing call on this thread ("" if none). */
const char *gk_last_error(void);

/* Library version string. */
const char *gk_version(void);

/* Launch plan of the matrix-core route for a product in the kernel frame (M x N
 * output, K bytes per operand row; in: 0 int8, 1 bf16, 2 f32; kind: 0 i32,
 * 1 f32, 2 bf16, 3 requantized i8/u8 output; ld_b: B^T's row stride in bytes,
 * 0 for rows of K bytes rounded up to 16), as the dispatcher would choose
 * it with the current environment: *tile is the tile of the (first) launch,
 * *na the kernel-frame columns it covers when the product is split into two
 * launches (else 0), *tile_b the tile of the second launch, *pn_a and *pn_b
 * (either may be NULL) the two launches' column pitches (0: the tile's
 * width).  Host-only, no device needed.  No counterpart in the reference: it
 * exposes the tile choice to tests and tuning tools. */
int gk_debug_plan(int32_t in, int32_t kind, int64_t m, int64_t n, int64_t batch, int64_t kbytes,
                  int64_t ld_b, int32_t *tile, int64_t *na, int32_t *tile_b, int32_t *pn_a,
                  int32_t *pn_b);

/* ---------------------------------------------------------------- runtime */

/* Parallelism request (src/parallel.rs:25): 1 = Serial, 0 = Rayon(0) "all",
 * n = Rayon(n).  Accepted for drop-in compatibility and ignored: the device
 * grid decides. */
typedef uint32_t gk_par;
#define GK_PAR_SERIAL 1u
#define GK_PAR_ALL 0u

/* bf16 values travel as their 16-bit patterns. */
typedef uint16_t gk_bf16;

/* Initialise the HIP device (called lazily by every entry point). */
int gk_init(void);

/* Stream the calling thread's launches go to (a hipStream_t; NULL = the null
 * stream).  Thread-local. */
int gk_set_stream(void *hip_stream);
void *gk_get_stream(void);

/* 1 (default): every call waits for its kernels, as the reference's synchronous
 * entry points do.  0: calls only enqueue.  Thread-local. */
int gk_set_synchronous(int on);

/* Device scratch arena (src/workspace.rs:53): holds packed operands for
 * layouts the kernels cannot read in place and split-K partial sums.  Grows on
 * demand (synchronizing the device), never shrinks.  A call made while the
 * launch stream is being captured into a HIP graph cannot grow it: such a call
 * fails with GK_ERR_NOMEM when it needs more than the arena holds, so size the
 * arena before capturing.  The NULL (per-thread) workspace is released when its
 * worker thread exits. */
typedef struct gk_workspace gk_workspace;
gk_workspace *gk_workspace_new(void);
/* Workspace::with_capacity (src/workspace.rs:78): an arena of at least `bytes`
 * allocated now; NULL when the device allocation fails. */
gk_workspace *gk_workspace_with_capacity(size_t bytes);
void gk_workspace_free(gk_workspace *ws);
size_t gk_workspace_bytes(const gk_workspace *ws);

/* ------------------------------------------------------------------ views */

/* MatRef / MatMut (src/api.rs:92-180): element (i, j) lives at
 * data + i*rs + j*cs; `len` is the backing slice length in elements. */
typedef struct gk_mat_ref {
    const void *data;
    size_t len;
    size_t rows;
    size_t cols;
    ptrdiff_t rs;
    ptrdiff_t cs;
} gk_mat_ref;

typedef struct gk_mat_mut {
    void *data;
    size_t len;
    size_t rows;
    size_t cols;
    ptrdiff_t rs;
    ptrdiff_t cs;
} gk_mat_mut;

/* --------------------------------------------------------- plain GEMM: f32 */

/* gemm::<f32> / gemm_with (src/api.rs:400, :418): C <- alpha*A*B + beta*C.
 * beta == 0 never reads C.  m == 1 or n == 1 takes the GEMV route, as
 * dispatch/float.rs:81 does. */
int gk_gemm_f32(gk_workspace *ws, float alpha, const gk_mat_ref *a, const gk_mat_ref *b,
                float beta, const gk_mat_mut *c, gk_par par);

/* gemm_unchecked::<f32> / gemm_unchecked_with (src/api.rs:469, :544). */
int gk_gemm_f32_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, float alpha,
                          const float *a, ptrdiff_t rsa, ptrdiff_t csa,
                          const float *b, ptrdiff_t rsb, ptrdiff_t csb,
                          float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par par);

/* -------------------------------------------------------- plain GEMM: bf16 */

/* gemm::<bf16> (src/api.rs:400 with GemmScalar for bf16, src/dispatch/mixed.rs:1395):
 * bf16 inputs, f32 accumulation, alpha*acc + beta*C in f32, one RNE narrowing to
 * bf16 (NaN -> (bits>>16)|0x40).  alpha/beta are bf16 like the reference's. */
int gk_gemm_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_mat_ref *a, const gk_mat_ref *b,
                 gk_bf16 beta, const gk_mat_mut *c, gk_par par);
int gk_gemm_bf16_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, gk_bf16 alpha,
                           const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa,
                           const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb,
                           gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par par);

/* Extension (no reference counterpart; the reference's bf16 GEMM always
 * narrows): bf16 inputs, f32 accumulation, f32 alpha/beta and f32 output C.
 * Same validation as gemm::<bf16>. */
int gk_gemm_bf16_f32out(gk_workspace *ws, float alpha, const gk_mat_ref *a,
                        const gk_mat_ref *b, float beta, const gk_mat_mut *c, gk_par par);
int gk_gemm_bf16_f32out_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, float alpha,
                                  const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa,
                                  const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb,
                                  float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc,
                                  gk_par par);

/* ------------------------------------------------------------- i8 -> i32 */

/* gemm_i8 / gemm_i8_with (src/api/int8.rs:22, :38): i8 inputs, i32 alpha/beta/C,
 * all arithmetic wrapping i32. */
int gk_gemm_i8(gk_workspace *ws, int32_t alpha, const gk_mat_ref *a, const gk_mat_ref *b,
               int32_t beta, const gk_mat_mut *c, gk_par par);

/* gemm_i8_unchecked / gemm_i8_unchecked_with (src/api/int8.rs:86, :136). */
int gk_gemm_i8_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, int32_t alpha,
                         const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                         const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
                         int32_t beta, int32_t *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par par);

/* No counterpart in the reference: gk_gemm_i8_unchecked for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments (no workspace), same
 * kernels and bit-identical results; packed operands and split-K partial sums
 * go to a static scratch of 64 MiB per device, held from module load to
 * process exit, instead of a workspace.  It calls no allocator.  A product
 * that needs more scratch than that fails with GK_ERR_NOMEM before launching
 * anything.  Every call on a device shares that device's scratch, so calls
 * that overlap on one device (other threads, other streams) race. */
int gk_gemm_i8_unchecked_noalloc(size_t m, size_t k, size_t n, int32_t alpha,
                                 const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                                 const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
                                 int32_t beta, int32_t *c, ptrdiff_t rsc, ptrdiff_t csc,
                                 gk_par par);

/* --------------------------------------------------------- requantization */

/* Channel axis of a requant scale vector / bias.  GK_AXIS_ROW is the
 * reference's only choice (RequantScale::PerRow, Requantize::bias, length m,
 * src/api/int8.rs:185-209); GK_AXIS_COL (length n, per output column) is an
 * extension of this engine. */
#define GK_AXIS_ROW 0
#define GK_AXIS_COL 1

/* Activation after requantization.  GK_ACT_RELU is an extension: it clamps the
 * quantized value below at max(LO, zero_point), which equals quantizing
 * max(0, real value) because round-half-even is monotone with rne(0) = 0. */
#define GK_ACT_NONE 0
#define GK_ACT_RELU 1
/* Fused-epilogue entries only (Activation::LeakyRelu, src/api/fused.rs:26-31). */
#define GK_ACT_LEAKY_RELU 2

/* Requantize (src/api/int8.rs:185-209) plus the two extension fields.
 * scales == NULL selects RequantScale::PerTensor(scale); otherwise `scales`
 * (device, scales_len entries) is the per-channel vector.  bias == NULL means
 * no bias.  Output: clamp(zp + round_half_even(scale*(acc + bias)), LO, HI). */
typedef struct gk_requantize {
    float scale;
    const float *scales;
    size_t scales_len;
    int32_t zero_point;
    const int32_t *bias;
    size_t bias_len;
    int32_t axis; /* GK_AXIS_ROW or GK_AXIS_COL */
    int32_t act;  /* GK_ACT_NONE or GK_ACT_RELU  */
} gk_requantize;

/* gemm_i8_requant / _with (src/api/int8.rs:230, :280): i8 output, LO/HI = -128/127.
 * The per-channel scales are checked (finite, > 0) by copying them to the host,
 * as the reference checks them when its RequantScale is built.  Under HIP graph
 * capture nothing can be copied back: a captured call accepts a scale vector
 * only when an uncaptured call on the same thread has checked one with the same
 * device pointer and length (the last 64 are remembered), and fails otherwise.
 * The match is by address: if the caller rewrites that buffer with invalid
 * scales, or frees it and gets the same address back, a captured call does not
 * see it (the reference's borrow of the slice makes that impossible there). */
int gk_gemm_i8_requant(gk_workspace *ws, const gk_mat_ref *a, const gk_mat_ref *b,
                       const gk_requantize *req, const gk_mat_mut *c, gk_par par);

/* gemm_i8_requant_u8 / _with (src/api/int8.rs:479, :510): u8 output, LO/HI = 0/255. */
int gk_gemm_i8_requant_u8(gk_workspace *ws, const gk_mat_ref *a, const gk_mat_ref *b,
                          const gk_requantize *req, const gk_mat_mut *c, gk_par par);

/* gemm_i8_requant_unchecked(_with) (src/api/int8.rs:347, :410) and the u8 twins
 * (:562, :615), with the axis/act extension arguments appended (pass
 * GK_AXIS_ROW, GK_ACT_NONE for the reference's behaviour). */
int gk_gemm_i8_requant_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n,
                                 const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                                 const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
                                 float scale, const float *row_scales, uint8_t has_row_scales,
                                 int32_t zero_point, const int32_t *bias, uint8_t has_bias,
                                 int8_t *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par par,
                                 int32_t axis, int32_t act);
int gk_gemm_i8_requant_u8_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n,
                                    const int8_t *a, ptrdiff_t rsa, ptrdiff_t csa,
                                    const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb,
                                    float scale, const float *row_scales,
                                    uint8_t has_row_scales, int32_t zero_point,
                                    const int32_t *bias, uint8_t has_bias,
                                    uint8_t *c, ptrdiff_t rsc, ptrdiff_t csc, gk_par par,
                                    int32_t axis, int32_t act);

/* -------------------------------------------------------- prepacked i8 RHS */

/* PackedRhs<i8> (src/api/packed.rs:34-52): an opaque, read-only device copy of
 * B in the kernels' k-contiguous tile layout; it can be shared by concurrent
 * calls and is released with gk_packed_rhs_free. */
typedef struct gk_packed_rhs gk_packed_rhs;

/* prepack_rhs_i8 (src/api/packed.rs:372): B is a device view (k x n). */
int gk_prepack_rhs_i8(const gk_mat_ref *b, gk_packed_rhs **out);
/* prepack_rhs_i8_unchecked (src/api/packed.rs:406). */
int gk_prepack_rhs_i8_unchecked(const int8_t *b, ptrdiff_t rsb, ptrdiff_t csb, size_t k,
                                size_t n, gk_packed_rhs **out);
void gk_packed_rhs_free(gk_packed_rhs *p);
/* PackedRhs::rows / cols (src/api/packed.rs:43-51). */
size_t gk_packed_rhs_rows(const gk_packed_rhs *p);
size_t gk_packed_rhs_cols(const gk_packed_rhs *p);

/* gemm_i8_packed_b / _with (src/api/packed.rs:473, :494): bit-identical to
 * gemm_i8; like the reference it requires a column-major-ish C
 * (|csc| >= |rsc|). */
int gk_gemm_i8_packed_b(gk_workspace *ws, int32_t alpha, const gk_mat_ref *a,
                        const gk_packed_rhs *packed, int32_t beta, const gk_mat_mut *c,
                        gk_par par);
/* gemm_i8_packed_b_unchecked(_with) (src/api/packed.rs:575, :612). */
int gk_gemm_i8_packed_b_unchecked(gk_workspace *ws, int32_t alpha, size_t m, const int8_t *a,
                                  ptrdiff_t rsa, ptrdiff_t csa, const gk_packed_rhs *packed,
                                  int32_t beta, int32_t *c, ptrdiff_t rsc, ptrdiff_t csc,
                                  gk_par par);

/* Extension (the reference has no prepacked requant entry): requantizing GEMM
 * against a prepacked B, i8 or u8 output, any C orientation.  Validation as
 * gk_gemm_i8_requant with B's shape taken from `packed`. */
int gk_gemm_i8_packed_b_requant(gk_workspace *ws, const gk_mat_ref *a,
                                const gk_packed_rhs *packed, const gk_requantize *req,
                                const gk_mat_mut *c, gk_par par);
int gk_gemm_i8_packed_b_requant_u8(gk_workspace *ws, const gk_mat_ref *a,
                                   const gk_packed_rhs *packed, const gk_requantize *req,
                                   const gk_mat_mut *c, gk_par par);
/* Unchecked twins of the two entries above (raw A/C pointers and strides, the
 * requant fields as gk_gemm_i8_requant_unchecked takes them); no validation. */
int gk_gemm_i8_packed_b_requant_unchecked(gk_workspace *ws, size_t m, const int8_t *a,
                                          ptrdiff_t rsa, ptrdiff_t csa,
                                          const gk_packed_rhs *packed, float scale,
                                          const float *scales, uint8_t has_scales,
                                          int32_t zero_point, const int32_t *bias,
                                          uint8_t has_bias, int8_t *c, ptrdiff_t rsc,
                                          ptrdiff_t csc, gk_par par, int32_t axis, int32_t act);
int gk_gemm_i8_packed_b_requant_u8_unchecked(gk_workspace *ws, size_t m, const int8_t *a,
                                             ptrdiff_t rsa, ptrdiff_t csa,
                                             const gk_packed_rhs *packed, float scale,
                                             const float *scales, uint8_t has_scales,
                                             int32_t zero_point, const int32_t *bias,
                                             uint8_t has_bias, uint8_t *c, ptrdiff_t rsc,
                                             ptrdiff_t csc, gk_par par, int32_t axis,
                                             int32_t act);

/* ------------------------------------------------------ prepacked f32/bf16 RHS */

/* prepack_rhs::<f32> / ::<bf16> (src/api/packed.rs:67) and prepack_rhs_unchecked
 * (:80): the same opaque handle as the i8 pack, typed by its element; an entry
 * given a handle of another element type returns GK_ERR_ARG. */
int gk_prepack_rhs_f32(const gk_mat_ref *b, gk_packed_rhs **out);
int gk_prepack_rhs_f32_unchecked(const float *b, ptrdiff_t rsb, ptrdiff_t csb, size_t k,
                                 size_t n, gk_packed_rhs **out);
int gk_prepack_rhs_bf16(const gk_mat_ref *b, gk_packed_rhs **out);
int gk_prepack_rhs_bf16_unchecked(const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb, size_t k,
                                  size_t n, gk_packed_rhs **out);

/* gemm_packed_b::<f32|bf16> / _with (src/api/packed.rs:175, :191): results as
 * gemm; a column-major-ish C (|csc| >= |rsc|) is required, as in the reference. */
int gk_gemm_packed_b_f32(gk_workspace *ws, float alpha, const gk_mat_ref *a,
                         const gk_packed_rhs *packed, float beta, const gk_mat_mut *c,
                         gk_par par);
/* gemm_packed_b_unchecked(_with) (src/api/packed.rs:270, :301). */
int gk_gemm_packed_b_f32_unchecked(gk_workspace *ws, float alpha, size_t m, const float *a,
                                   ptrdiff_t rsa, ptrdiff_t csa, const gk_packed_rhs *packed,
                                   float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc,
                                   gk_par par);
int gk_gemm_packed_b_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_mat_ref *a,
                          const gk_packed_rhs *packed, gk_bf16 beta, const gk_mat_mut *c,
                          gk_par par);
int gk_gemm_packed_b_bf16_unchecked(gk_workspace *ws, gk_bf16 alpha, size_t m, const gk_bf16 *a,
                                    ptrdiff_t rsa, ptrdiff_t csa, const gk_packed_rhs *packed,
                                    gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc, ptrdiff_t csc,
                                    gk_par par);

/* ----------------------------------------------------------- batched GEMM */

/* gemm_batched::<f32> / _with (src/api/batched.rs:188, :225): element bi uses
 * A + bi*a_bs, B + bi*b_bs, C + bi*c_bs (element strides; 0 broadcasts A or B). */
int gk_gemm_batched_f32(gk_workspace *ws, size_t batch, float alpha,
                        const gk_mat_ref *a, ptrdiff_t a_bs,
                        const gk_mat_ref *b, ptrdiff_t b_bs, float beta,
                        const gk_mat_mut *c, ptrdiff_t c_bs, gk_par par);
/* gemm_batched_unchecked(_with) (src/api/batched.rs:594, :649). */
int gk_gemm_batched_f32_unchecked(gk_workspace *ws, size_t batch, size_t m, size_t k,
                                  size_t n, float alpha,
                                  const float *a, ptrdiff_t rsa, ptrdiff_t csa, ptrdiff_t a_bs,
                                  const float *b, ptrdiff_t rsb, ptrdiff_t csb, ptrdiff_t b_bs,
                                  float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc,
                                  ptrdiff_t c_bs, gk_par par);

/* gemm_batched::<bf16> (src/api/batched.rs:188): bf16 in and out. */
int gk_gemm_batched_bf16(gk_workspace *ws, size_t batch, gk_bf16 alpha,
                         const gk_mat_ref *a, ptrdiff_t a_bs,
                         const gk_mat_ref *b, ptrdiff_t b_bs, gk_bf16 beta,
                         const gk_mat_mut *c, ptrdiff_t c_bs, gk_par par);
int gk_gemm_batched_bf16_unchecked(gk_workspace *ws, size_t batch, size_t m, size_t k,
                                   size_t n, gk_bf16 alpha,
                                   const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa,
                                   ptrdiff_t a_bs, const gk_bf16 *b, ptrdiff_t rsb,
                                   ptrdiff_t csb, ptrdiff_t b_bs, gk_bf16 beta, gk_bf16 *c,
                                   ptrdiff_t rsc, ptrdiff_t csc, ptrdiff_t c_bs, gk_par par);

/* Extension: batched bf16 x bf16 with f32 accumulation and f32 alpha/beta/C
 * (the attention-score shape); validation as gemm_batched. */
int gk_gemm_batched_bf16_f32out(gk_workspace *ws, size_t batch, float alpha,
                                const gk_mat_ref *a, ptrdiff_t a_bs,
                                const gk_mat_ref *b, ptrdiff_t b_bs, float beta,
                                const gk_mat_mut *c, ptrdiff_t c_bs, gk_par par);
int gk_gemm_batched_bf16_f32out_unchecked(gk_workspace *ws, size_t batch, size_t m, size_t k,
                                          size_t n, float alpha,
                                          const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa,
                                          ptrdiff_t a_bs, const gk_bf16 *b, ptrdiff_t rsb,
                                          ptrdiff_t csb, ptrdiff_t b_bs, float beta, float *c,
                                          ptrdiff_t rsc, ptrdiff_t csc, ptrdiff_t c_bs,
                                          gk_par par);

/* ------------------------------------------ pointer-array batched GEMM */

/* GemmProblem (src/dispatch.rs:135-164): one independent product with its own
 * shape, scalars, device pointers and strides. */
typedef struct gk_problem_f32 {
    size_t m, k, n;
    float alpha;
    const float *a;
    ptrdiff_t rsa, csa;
    const float *b;
    ptrdiff_t rsb, csb;
    float beta;
    float *c;
    ptrdiff_t rsc, csc;
} gk_problem_f32;

typedef struct gk_problem_bf16 {
    size_t m, k, n;
    gk_bf16 alpha;
    const gk_bf16 *a;
    ptrdiff_t rsa, csa;
    const gk_bf16 *b;
    ptrdiff_t rsb, csb;
    gk_bf16 beta;
    gk_bf16 *c;
    ptrdiff_t rsc, csc;
} gk_problem_bf16;

/* gemm_batched_ptr_unchecked (src/api/batched.rs:711-720): every problem of
 * the host array runs as the standalone gemm would (bit for bit).  Runs of
 * consecutive problems with one shape, one set of scalars and strides and
 * constant pointer steps go out as one strided batched launch.  The caller
 * guarantees what the reference's Safety section asks: valid pointers,
 * outputs pairwise disjoint and aliasing no input. */
int gk_gemm_batched_ptr_f32_unchecked(gk_workspace *ws, const gk_problem_f32 *problems,
                                      size_t count, gk_par par);
int gk_gemm_batched_ptr_bf16_unchecked(gk_workspace *ws, const gk_problem_bf16 *problems,
                                       size_t count, gk_par par);

/* BatchProblem (src/api/batched.rs:723-735): one element of the checked form. */
typedef struct gk_batch_problem_f32 {
    float alpha;
    gk_mat_ref a;
    gk_mat_ref b;
    float beta;
    gk_mat_mut c;
} gk_batch_problem_f32;

typedef struct gk_batch_problem_bf16 {
    gk_bf16 alpha;
    gk_mat_ref a;
    gk_mat_ref b;
    gk_bf16 beta;
    gk_mat_mut c;
} gk_batch_problem_bf16;

/* gemm_batched_slice (src/api/batched.rs:748-799): per element, the shape
 * agreement, view bounds and C self-alias checks with the reference's
 * messages ("gemmkit: batch element i ..."), then the pointer-array run.  In
 * the reference distinct &mut borrows make the outputs disjoint; here that is
 * the caller's guarantee, as for the raw form. */
int gk_gemm_batched_slice_f32(gk_workspace *ws, const gk_batch_problem_f32 *problems,
                              size_t count, gk_par par);
int gk_gemm_batched_slice_bf16(gk_workspace *ws, const gk_batch_problem_bf16 *problems,
                               size_t count, gk_par par);

/* --------------------------------------------- fused bias and activation */

/* Bias (src/api/fused.rs:17-23) / BiasDim (src/kernel/epilogue.rs:205-210):
 * one value per output row (length m) or per output column (length n),
 * added after alpha*A*B + beta*C and before the activation. */
#define GK_BIAS_PER_ROW 0
#define GK_BIAS_PER_COL 1

/* A checked-tier bias: `data` is a device float* (f32 entries) or gk_bf16*
 * (bf16 entries), `len` its length in elements, `dim` GK_BIAS_PER_ROW or
 * GK_BIAS_PER_COL.  A NULL gk_bias* is Option::None. */
typedef struct gk_bias {
    const void *data;
    size_t len;
    int32_t dim;
} gk_bias;

/* Semantics of every fused entry (FusedEpi::apply, src/kernel/epilogue.rs:309-330
 * and :569-596): C <- act(alpha*A*B + beta*C + bias), act = GK_ACT_NONE,
 * GK_ACT_RELU (v > 0 ? v : 0) or GK_ACT_LEAKY_RELU (max(v,0) + slope*min(v,0));
 * NaN and -0 map to +0.  f32: bit-identical to the plain GEMM followed by the
 * same scalar map.  bf16: the map runs in f32 on the accumulator (bias and
 * slope widened exactly), then one RNE narrowing.  Checked entries add the
 * reference's bias checks ("gemmkit: PerRow bias length (..) != A.rows (..)",
 * "... PerCol ... != B.cols", "gemmkit: bias slice overlaps C") and
 * "gemmkit: LeakyRelu slope must be finite"; with no bias and no activation
 * they are the plain GEMM.  The unchecked entries take the reference's raw
 * (bias, bias_dim, has_bias) triple and the activation as (act, slope). */

/* gemm_fused::<f32|bf16> / _with (src/api/fused.rs:61, :81). */
int gk_gemm_fused_f32(gk_workspace *ws, float alpha, const gk_mat_ref *a, const gk_mat_ref *b,
                      float beta, const gk_mat_mut *c, const gk_bias *bias, int32_t act,
                      float slope, gk_par par);
int gk_gemm_fused_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_mat_ref *a, const gk_mat_ref *b,
                       gk_bf16 beta, const gk_mat_mut *c, const gk_bias *bias, int32_t act,
                       gk_bf16 slope, gk_par par);
/* gemm_fused_unchecked(_with) (src/api/fused.rs:149, :184). */
int gk_gemm_fused_f32_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, float alpha,
                                const float *a, ptrdiff_t rsa, ptrdiff_t csa,
                                const float *b, ptrdiff_t rsb, ptrdiff_t csb,
                                float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc,
                                const float *bias, int32_t bias_dim, uint8_t has_bias,
                                int32_t act, float slope, gk_par par);
int gk_gemm_fused_bf16_unchecked(gk_workspace *ws, size_t m, size_t k, size_t n, gk_bf16 alpha,
                                 const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa,
                                 const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb,
                                 gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc, ptrdiff_t csc,
                                 const gk_bf16 *bias, int32_t bias_dim, uint8_t has_bias,
                                 int32_t act, gk_bf16 slope, gk_par par);

/* gemm_batched_fused / _with (src/api/batched.rs:307, :348): one shared bias
 * vector, sized for a single element, and one activation for every element. */
int gk_gemm_batched_fused_f32(gk_workspace *ws, size_t batch, float alpha,
                              const gk_mat_ref *a, ptrdiff_t a_bs,
                              const gk_mat_ref *b, ptrdiff_t b_bs, float beta,
                              const gk_mat_mut *c, ptrdiff_t c_bs, const gk_bias *bias,
                              int32_t act, float slope, gk_par par);
int gk_gemm_batched_fused_bf16(gk_workspace *ws, size_t batch, gk_bf16 alpha,
                               const gk_mat_ref *a, ptrdiff_t a_bs,
                               const gk_mat_ref *b, ptrdiff_t b_bs, gk_bf16 beta,
                               const gk_mat_mut *c, ptrdiff_t c_bs, const gk_bias *bias,
                               int32_t act, gk_bf16 slope, gk_par par);
/* gemm_batched_fused_unchecked(_with) (src/api/batched.rs:459, :523). */
int gk_gemm_batched_fused_f32_unchecked(gk_workspace *ws, size_t batch, size_t m, size_t k,
                                        size_t n, float alpha,
                                        const float *a, ptrdiff_t rsa, ptrdiff_t csa,
                                        ptrdiff_t a_bs, const float *b, ptrdiff_t rsb,
                                        ptrdiff_t csb, ptrdiff_t b_bs, float beta, float *c,
                                        ptrdiff_t rsc, ptrdiff_t csc, ptrdiff_t c_bs,
                                        const float *bias, int32_t bias_dim, uint8_t has_bias,
                                        int32_t act, float slope, gk_par par);
int gk_gemm_batched_fused_bf16_unchecked(gk_workspace *ws, size_t batch, size_t m, size_t k,
                                         size_t n, gk_bf16 alpha,
                                         const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa,
                                         ptrdiff_t a_bs, const gk_bf16 *b, ptrdiff_t rsb,
                                         ptrdiff_t csb, ptrdiff_t b_bs, gk_bf16 beta, gk_bf16 *c,
                                         ptrdiff_t rsc, ptrdiff_t csc, ptrdiff_t c_bs,
                                         const gk_bf16 *bias, int32_t bias_dim,
                                         uint8_t has_bias, int32_t act, gk_bf16 slope,
                                         gk_par par);

/* gemm_packed_b_fused / _with (src/api/packed.rs:684, :706): the checks of
 * gemm_packed_b plus the bias checks; column-major-ish C required. */
int gk_gemm_packed_b_fused_f32(gk_workspace *ws, float alpha, const gk_mat_ref *a,
                               const gk_packed_rhs *packed, float beta, const gk_mat_mut *c,
                               const gk_bias *bias, int32_t act, float slope, gk_par par);
int gk_gemm_packed_b_fused_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_mat_ref *a,
                                const gk_packed_rhs *packed, gk_bf16 beta, const gk_mat_mut *c,
                                const gk_bias *bias, int32_t act, gk_bf16 slope, gk_par par);
/* gemm_packed_b_fused_unchecked(_with) (src/api/packed.rs:801, :838). */
int gk_gemm_packed_b_fused_f32_unchecked(gk_workspace *ws, float alpha, size_t m, const float *a,
                                         ptrdiff_t rsa, ptrdiff_t csa,
                                         const gk_packed_rhs *packed, float beta, float *c,
                                         ptrdiff_t rsc, ptrdiff_t csc, const float *bias,
                                         int32_t bias_dim, uint8_t has_bias, int32_t act,
                                         float slope, gk_par par);
int gk_gemm_packed_b_fused_bf16_unchecked(gk_workspace *ws, gk_bf16 alpha, size_t m,
                                          const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa,
                                          const gk_packed_rhs *packed, gk_bf16 beta, gk_bf16 *c,
                                          ptrdiff_t rsc, ptrdiff_t csc, const gk_bf16 *bias,
                                          int32_t bias_dim, uint8_t has_bias, int32_t act,
                                          gk_bf16 slope, gk_par par);

/* ---------------------------------------------------- prepacked float LHS */

/* PackedLhs<T> (src/api/packed.rs:953-981): an opaque, read-only device copy
 * of A (m x k) in the kernels' k-contiguous row layout, for f32 or bf16;
 * released with gk_packed_lhs_free. */
typedef struct gk_packed_lhs gk_packed_lhs;

/* prepack_lhs (src/api/packed.rs:986) / prepack_lhs_unchecked (:999). */
int gk_prepack_lhs_f32(const gk_mat_ref *a, gk_packed_lhs **out);
int gk_prepack_lhs_f32_unchecked(const float *a, ptrdiff_t rsa, ptrdiff_t csa, size_t m,
                                 size_t k, gk_packed_lhs **out);
int gk_prepack_lhs_bf16(const gk_mat_ref *a, gk_packed_lhs **out);
int gk_prepack_lhs_bf16_unchecked(const gk_bf16 *a, ptrdiff_t rsa, ptrdiff_t csa, size_t m,
                                  size_t k, gk_packed_lhs **out);
void gk_packed_lhs_free(gk_packed_lhs *p);
/* PackedLhs::rows / cols (src/api/packed.rs:963-973). */
size_t gk_packed_lhs_rows(const gk_packed_lhs *p);
size_t gk_packed_lhs_cols(const gk_packed_lhs *p);

/* gemm_packed_a / _with (src/api/packed.rs:1049, :1065): C <- alpha*A*B +
 * beta*C with the prepacked A, bit-identical to gemm; like the reference it
 * requires a row-major-ish C (|csc| <= |rsc|). */
int gk_gemm_packed_a_f32(gk_workspace *ws, float alpha, const gk_packed_lhs *packed,
                         const gk_mat_ref *b, float beta, const gk_mat_mut *c, gk_par par);
int gk_gemm_packed_a_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_packed_lhs *packed,
                          const gk_mat_ref *b, gk_bf16 beta, const gk_mat_mut *c, gk_par par);
/* gemm_packed_a_unchecked(_with) (src/api/packed.rs:1143, :1174). */
int gk_gemm_packed_a_f32_unchecked(gk_workspace *ws, float alpha, const gk_packed_lhs *packed,
                                   size_t n, const float *b, ptrdiff_t rsb, ptrdiff_t csb,
                                   float beta, float *c, ptrdiff_t rsc, ptrdiff_t csc,
                                   gk_par par);
int gk_gemm_packed_a_bf16_unchecked(gk_workspace *ws, gk_bf16 alpha, const gk_packed_lhs *packed,
                                    size_t n, const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb,
                                    gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc, ptrdiff_t csc,
                                    gk_par par);
/* gemm_packed_a_fused / _with (src/api/packed.rs:1250, :1272): the checks of
 * gemm_packed_a plus the bias checks (bias in the user frame). */
int gk_gemm_packed_a_fused_f32(gk_workspace *ws, float alpha, const gk_packed_lhs *packed,
                               const gk_mat_ref *b, float beta, const gk_mat_mut *c,
                               const gk_bias *bias, int32_t act, float slope, gk_par par);
int gk_gemm_packed_a_fused_bf16(gk_workspace *ws, gk_bf16 alpha, const gk_packed_lhs *packed,
                                const gk_mat_ref *b, gk_bf16 beta, const gk_mat_mut *c,
                                const gk_bias *bias, int32_t act, gk_bf16 slope, gk_par par);
/* gemm_packed_a_fused_unchecked(_with) (src/api/packed.rs:1369, :1406). */
int gk_gemm_packed_a_fused_f32_unchecked(gk_workspace *ws, float alpha,
                                         const gk_packed_lhs *packed, size_t n, const float *b,
                                         ptrdiff_t rsb, ptrdiff_t csb, float beta, float *c,
                                         ptrdiff_t rsc, ptrdiff_t csc, const float *bias,
                                         int32_t bias_dim, uint8_t has_bias, int32_t act,
                                         float slope, gk_par par);
int gk_gemm_packed_a_fused_bf16_unchecked(gk_workspace *ws, gk_bf16 alpha,
                                          const gk_packed_lhs *packed, size_t n,
                                          const gk_bf16 *b, ptrdiff_t rsb, ptrdiff_t csb,
                                          gk_bf16 beta, gk_bf16 *c, ptrdiff_t rsc, ptrdiff_t csc,
                                          const gk_bf16 *bias, int32_t bias_dim,
                                          uint8_t has_bias, int32_t act, gk_bf16 slope,
                                          gk_par par);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* GEMMKIT_HIP_H */
