/* kurumi_hip C ABI: the MI355X (gfx950) backend for kurumi graphs.
 *
 * The graph-builder, eval, feeds, tensor, inspection and plan entry points keep the names,
 * argument meaning and error conventions of the reference header
 * (reference: kurumi/include/kurumi.h; each prototype below cites the line it mirrors), so a
 * frontend written against kurumi.h links against libkurumi_hip.so unchanged for this subset.
 * Conventions: builders return a node id or KU_ERR (then ku_last_error()); pointer-returning
 * calls return NULL on error; int-returning calls return 0 / -1. Handles are opaque and freed
 * with their ku_*_free. Not thread-safe per handle (kurumi.h:5).
 *
 * Backend kinds: KU_CPU (0) is the reference interpreter and lives in kurumi itself; this
 * library provides KU_HIP (2) only. Every op a KU_HIP backend accepts runs on the GPU; an op
 * outside its scope makes eval fail with an error (there is no CPU fallback).
 *
 * Entry points prefixed ku_hip_ have no counterpart in kurumi.h: device-resident plans for
 * benchmarking/serving, profile counters and codegen introspection. */
#ifndef KURUMI_HIP_H
#define KURUMI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KU_ERR 0xFFFFFFFFu /* kurumi.h:25 */

/* kurumi.h:29-34 (index = kurumi DType declaration order) */
typedef enum {
  KU_BOOL = 0, KU_U8, KU_U16, KU_U32, KU_U64,
  KU_I8, KU_I16, KU_I32, KU_I64,
  KU_F8E4M3, KU_F8E5M2, KU_F16, KU_BF16, KU_F32, KU_F64,
  KU_C64, KU_C128
} KuDType;

/* kurumi.h:38, plus KU_HIP */
typedef enum { KU_CPU = 0, KU_METAL = 1, KU_HIP = 2 } KuBackendKind;

typedef struct KuGraph KuGraph;
typedef struct KuTensor KuTensor;
typedef struct KuFeeds KuFeeds;
typedef struct KuBackend KuBackend;
typedef struct KuPlan KuPlan;
typedef struct KuHipPlan KuHipPlan;
typedef struct KuRunnable KuRunnable;
typedef uint32_t KuNode;

const char *ku_last_error(void); /* kurumi.h:51 */

/* graph lifecycle and leaves: kurumi.h:54-60 */
KuGraph *ku_graph_new(void);
void ku_graph_free(KuGraph *g);
KuNode ku_input(KuGraph *g, const size_t *shape, size_t rank, uint32_t dtype);
KuNode ku_constant_f32(KuGraph *g, const float *data, size_t len, const size_t *shape, size_t rank);
KuNode ku_constant(KuGraph *g, uint32_t dtype, const uint8_t *data, size_t nbytes, const size_t *shape, size_t rank);
KuNode ku_scalar(KuGraph *g, KuNode like, float v);

/* two-operand builders: kurumi.h:63-80 */
KuNode ku_add(KuGraph *g, KuNode a, KuNode b);
KuNode ku_sub(KuGraph *g, KuNode a, KuNode b);
KuNode ku_mul(KuGraph *g, KuNode a, KuNode b);
KuNode ku_div(KuGraph *g, KuNode a, KuNode b);
KuNode ku_max(KuGraph *g, KuNode a, KuNode b);
KuNode ku_idiv(KuGraph *g, KuNode a, KuNode b);
KuNode ku_and(KuGraph *g, KuNode a, KuNode b);
KuNode ku_or(KuGraph *g, KuNode a, KuNode b);
KuNode ku_xor(KuGraph *g, KuNode a, KuNode b);
KuNode ku_shl(KuGraph *g, KuNode a, KuNode b);
KuNode ku_shr(KuGraph *g, KuNode a, KuNode b);
KuNode ku_lt(KuGraph *g, KuNode a, KuNode b);
KuNode ku_eq(KuGraph *g, KuNode a, KuNode b);
KuNode ku_where(KuGraph *g, KuNode cond, KuNode a, KuNode b); /* kurumi.h:244 */

/* unary builders: kurumi.h:101-127 */
KuNode ku_neg(KuGraph *g, KuNode x);
KuNode ku_recip(KuGraph *g, KuNode x);
KuNode ku_sqrt(KuGraph *g, KuNode x);
KuNode ku_square(KuGraph *g, KuNode x);
KuNode ku_abs(KuGraph *g, KuNode x);
KuNode ku_sign(KuGraph *g, KuNode x);  /* kurumi.h:106 */
KuNode ku_floor(KuGraph *g, KuNode x);
KuNode ku_ceil(KuGraph *g, KuNode x);  /* kurumi.h:108 */
KuNode ku_round(KuGraph *g, KuNode x); /* kurumi.h:109 */
KuNode ku_exp(KuGraph *g, KuNode x);
KuNode ku_exp2(KuGraph *g, KuNode x);
KuNode ku_ln(KuGraph *g, KuNode x);
KuNode ku_log2(KuGraph *g, KuNode x);
KuNode ku_sin(KuGraph *g, KuNode x);
KuNode ku_cos(KuGraph *g, KuNode x);
KuNode ku_relu(KuGraph *g, KuNode x);
KuNode ku_gelu(KuGraph *g, KuNode x);    /* kurumi.h:128 */
KuNode ku_silu(KuGraph *g, KuNode x);    /* kurumi.h:130 */
KuNode ku_sigmoid(KuGraph *g, KuNode x); /* kurumi.h:131 */
KuNode ku_tanh(KuGraph *g, KuNode x);    /* kurumi.h:132 */
KuNode ku_rope(KuGraph *g, KuNode x);    /* kurumi.h:183 */
KuNode ku_flatten(KuGraph *g, KuNode x); /* kurumi.h:160 */
KuNode ku_t(KuGraph *g, KuNode x);       /* kurumi.h:161 */
KuNode ku_sum_all(KuGraph *g, KuNode x); /* kurumi.h:165 */

/* reductions over one axis: kurumi.h:186-199 */
KuNode ku_sum(KuGraph *g, KuNode x, size_t axis);
KuNode ku_prod(KuGraph *g, KuNode x, size_t axis);
KuNode ku_mean(KuGraph *g, KuNode x, size_t axis);
KuNode ku_reduce_max(KuGraph *g, KuNode x, size_t axis);
KuNode ku_reduce_min(KuGraph *g, KuNode x, size_t axis);
KuNode ku_argmax(KuGraph *g, KuNode x, size_t axis);
KuNode ku_argmin(KuGraph *g, KuNode x, size_t axis);
KuNode ku_softmax(KuGraph *g, KuNode x, size_t axis);
KuNode ku_log_softmax(KuGraph *g, KuNode x, size_t axis); /* kurumi.h:201 */
KuNode ku_logsumexp(KuGraph *g, KuNode x, size_t axis);   /* kurumi.h:202 */
KuNode ku_squeeze(KuGraph *g, KuNode x, size_t axis);   /* kurumi.h:209 */
KuNode ku_unsqueeze(KuGraph *g, KuNode x, size_t axis); /* kurumi.h:210 */
KuNode ku_clamp_min(KuGraph *g, KuNode x, float v);     /* kurumi.h:217 */
KuNode ku_rmsnorm(KuGraph *g, KuNode x, size_t axis, float eps); /* kurumi.h:302 */

/* contraction: kurumi.h:221-224 */
KuNode ku_matmul(KuGraph *g, KuNode a, KuNode b);
KuNode ku_dot_general(KuGraph *g, KuNode a, KuNode b, const size_t *lc, size_t nlc, const size_t *rc, size_t nrc,
                      const size_t *lb, size_t nlb, const size_t *rb, size_t nrb);

/* weight-only quantized matmul: act[M,K] x dequant(qweight)[N,K]^T -> [M,N] (kurumi.h:225-234);
 * qweight KU_U8-packed, scales/mins KU_F16 [N, K/group_size], mins = KU_ERR for symmetric */
KuNode ku_quant_matmul(KuGraph *g, KuNode act, KuNode qweight, KuNode scales, KuNode mins, uint8_t bits,
                       size_t group_size);
void ku_quantize(const float *w, size_t rows, size_t cols, uint8_t bits, size_t group_size, uint32_t symmetric,
                 uint8_t *out_packed, uint16_t *out_scales, uint16_t *out_mins);

/* movement: kurumi.h:269-276, 286-292 */
KuNode ku_reshape(KuGraph *g, KuNode x, const size_t *shape, size_t rank);
KuNode ku_expand(KuGraph *g, KuNode x, const size_t *shape, size_t rank);
KuNode ku_permute(KuGraph *g, KuNode x, const size_t *perm, size_t rank);
KuNode ku_transpose(KuGraph *g, KuNode x, size_t i, size_t j);
KuNode ku_flip(KuGraph *g, KuNode x, const size_t *axes, size_t n);
KuNode ku_slice(KuGraph *g, KuNode x, const size_t *ranges, size_t rank);      /* 2*rank (start,end) */
KuNode ku_slice_step(KuGraph *g, KuNode x, const size_t *ranges, size_t rank); /* 3*rank (start,end,step) */
KuNode ku_pad(KuGraph *g, KuNode x, const size_t *pads, size_t rank);          /* 2*rank (lo,hi), 0 */
KuNode ku_broadcast_to(KuGraph *g, KuNode x, const size_t *shape, size_t rank);
KuNode ku_detach(KuGraph *g, KuNode x);
KuNode ku_iota(KuGraph *g, const size_t *shape, size_t rank, size_t axis, uint32_t dtype);
KuNode ku_cast(KuGraph *g, KuNode x, uint32_t dtype);
KuNode ku_bitcast(KuGraph *g, KuNode x, uint32_t dtype);

/* attention: kurumi.h:343 (auto-selects fused vs decomposed like the reference builder) */
KuNode ku_sdpa(KuGraph *g, KuNode q, KuNode k, KuNode v, uint32_t causal);
/* random: kurumi.h:346-350 */
KuNode ku_rand_uniform(KuGraph *g, const size_t *shape, size_t rank, uint64_t seed);
KuNode ku_randn(KuGraph *g, const size_t *shape, size_t rank, uint64_t seed);
KuNode ku_rand_range(KuGraph *g, const size_t *shape, size_t rank, uint64_t seed, float lo, float hi);

/* backend + eval: kurumi.h:381-388 */
KuBackend *ku_backend_new(uint32_t kind); /* NULL if unavailable */
void ku_backend_free(KuBackend *b);
KuTensor *ku_eval(KuGraph *g, KuNode node, const KuBackend *backend);
KuTensor *ku_eval_with(KuGraph *g, KuNode node, const KuBackend *backend, const KuFeeds *feeds);
int32_t ku_eval_many(KuGraph *g, const KuNode *ids, size_t n, const KuBackend *backend, const KuFeeds *feeds,
                     KuTensor **out);

/* inspection: kurumi.h:396-405 */
size_t ku_node_count(const KuGraph *g, KuNode root);
size_t ku_dump(const KuGraph *g, KuNode root, uint8_t *out, size_t cap);
size_t ku_node_rank(const KuGraph *g, KuNode node);
void ku_node_shape(const KuGraph *g, KuNode node, size_t *out);
uint32_t ku_node_dtype(const KuGraph *g, KuNode node);

/* runnable-graph serialization, KGPH v2 blobs: kurumi.h:407-453. Inputs bind by (node, role,
 * name): role 0 = weight (bound by name), 1 = runtime feed; in_names are NUL-terminated UTF-8.
 * Size-then-write: cap=0 with out=NULL returns the length (0 and ku_last_error on failure). */
size_t ku_graph_serialize(const KuGraph *g, const KuNode *outputs, size_t n_out, const KuNode *in_nodes,
                          const uint8_t *in_roles, const char *const *in_names, size_t n_in, uint8_t *out, size_t cap);
size_t ku_graph_serialize_reachable(const KuGraph *g, const KuNode *outputs, size_t n_out, const KuNode *in_nodes,
                                    const uint8_t *in_roles, const char *const *in_names, size_t n_in, uint8_t *out,
                                    size_t cap);
size_t ku_graph_serialize_multi(const KuGraph *g, size_t n_entries, const char *const *names,
                                const uint32_t *out_counts, const KuNode *outputs, const uint32_t *in_counts,
                                const KuNode *in_nodes, const uint8_t *in_roles, const char *const *in_names,
                                uint8_t *out, size_t cap);
/* NULL (see ku_last_error) on a malformed or entry-less blob; every node is replayed through
 * the checked builders. Ops outside this IR (linalg, complex, gather/scatter, argsort) are
 * rejected with their name; QuantMatmul (tag 40) decodes like any other op. */
KuRunnable *ku_graph_deserialize(const uint8_t *bytes, size_t len);
KuGraph *ku_runnable_take_graph(KuRunnable *h);
size_t ku_runnable_output_count(const KuRunnable *h);
KuNode ku_runnable_output(const KuRunnable *h, size_t i);
size_t ku_runnable_input_count(const KuRunnable *h);
KuNode ku_runnable_input_node(const KuRunnable *h, size_t i);
uint32_t ku_runnable_input_role(const KuRunnable *h, size_t i);
size_t ku_runnable_input_name(const KuRunnable *h, size_t i, uint8_t *out, size_t cap);
size_t ku_runnable_entry_count(const KuRunnable *h);
size_t ku_runnable_entry_name(const KuRunnable *h, size_t i, uint8_t *out, size_t cap);
size_t ku_runnable_entry_output_count(const KuRunnable *h, size_t i);
KuNode ku_runnable_entry_output(const KuRunnable *h, size_t i, size_t j);
size_t ku_runnable_entry_input_count(const KuRunnable *h, size_t i);
KuNode ku_runnable_entry_input_node(const KuRunnable *h, size_t i, size_t j);
uint32_t ku_runnable_entry_input_role(const KuRunnable *h, size_t i, size_t j);
size_t ku_runnable_entry_input_name(const KuRunnable *h, size_t i, size_t j, uint8_t *out, size_t cap);
void ku_runnable_free(KuRunnable *h);

/* plan-replay: kurumi.h:456-458. Here the plan is a device plan, replayed as one hipGraph
 * launch per run. ku_plan_compile has no backend argument, so its plans live on a
 * process-default KU_HIP backend (device 0) that is created on first use and never destroyed
 * (its device memory is returned when the process ends). ku_plan_run requires the graph the
 * plan was compiled on, or one with the same content. */
KuPlan *ku_plan_compile(const KuGraph *g, KuNode node);
KuTensor *ku_plan_run(const KuPlan *p, const KuGraph *g, const KuFeeds *feeds);
void ku_plan_free(KuPlan *p);

/* feeds: kurumi.h:461-463 */
KuFeeds *ku_feeds_new(void);
void ku_feeds_free(KuFeeds *f);
void ku_feeds_set(KuFeeds *f, KuNode node, const KuTensor *tensor);

/* tensors: kurumi.h:466-479 */
KuTensor *ku_tensor_f32(const float *data, size_t len, const size_t *shape, size_t rank);
KuTensor *ku_tensor_new(uint32_t dtype, const uint8_t *data, size_t nbytes, const size_t *shape, size_t rank);
void ku_tensor_free(KuTensor *t);
size_t ku_tensor_rank(const KuTensor *t);
void ku_tensor_shape(const KuTensor *t, size_t *out);
size_t ku_tensor_len(const KuTensor *t);
uint32_t ku_tensor_dtype(const KuTensor *t);
ptrdiff_t ku_tensor_data_f32(const KuTensor *t, float *out, size_t cap);
size_t ku_tensor_nbytes(const KuTensor *t);
void ku_tensor_bytes(const KuTensor *t, uint8_t *out);

/* ---- extensions without a kurumi.h counterpart ---- */

/* Explicit attention forms of the reference builders Graph::sdpa_decomposed / sdpa_fused
 * (kurumi_core/src/graph/ops/nn/attention.rs:97-133), which kurumi.h does not export. */
KuNode ku_sdpa_decomposed(KuGraph *g, KuNode q, KuNode k, KuNode v, uint32_t causal);
KuNode ku_sdpa_fused(KuGraph *g, KuNode q, KuNode k, KuNode v, uint32_t causal);

/* kurumi.h:395: the reference's mixed-precision pass (f16 matmuls): every f32 DotGeneral under
 * `root` takes f16 casts of its operands and is cast back to f32. Returns the new root. */
KuNode ku_amp(KuGraph *g, KuNode root);

/* fp8 (OCP e4m3) mixed-precision pass: rewrites linear DotGenerals under `root` into a
 * per-tensor-scaled activation x per-row-scaled weight e4m3 contraction (the e4m3 policy
 * next to kurumi.h:395 ku_amp, which is f16-only). Returns the new root or KU_ERR. */
KuNode ku_amp_fp8(KuGraph *g, KuNode root);

/* ku_plan_compile on a caller's backend, sharing its plan and constant caches; run and free
 * with ku_plan_run / ku_plan_free. The plan keeps the backend alive: ku_backend_free may come
 * before ku_plan_free, and the backend's device memory is released with its last plan. */
KuPlan *ku_hip_plan_compile_on(const KuBackend *b, const KuGraph *g, KuNode node);

/* Device-resident plan: compile `roots`, upload `feeds` once, then launch repeatedly with
 * inputs and outputs staying in HBM. The graph must outlive the plan; the backend need not (the
 * plan keeps it alive, as ku_hip_plan_compile_on's plans do). */
KuHipPlan *ku_hip_plan_new(KuGraph *g, const KuNode *roots, size_t n, const KuBackend *backend,
                           const KuFeeds *feeds);
int32_t ku_hip_plan_feed(KuHipPlan *p, KuNode input, const KuTensor *t);
int32_t ku_hip_plan_launch(KuHipPlan *p, uint32_t use_graph); /* async on the backend stream */
int32_t ku_hip_plan_sync(KuHipPlan *p);
KuTensor *ku_hip_plan_output(KuHipPlan *p, size_t i);
size_t ku_hip_plan_num_steps(const KuHipPlan *p);
/* NUL-terminated label of step i (kernel name / variant); copied into out (cap bytes). */
size_t ku_hip_plan_step_label(const KuHipPlan *p, size_t i, char *out, size_t cap);
/* Average GPU milliseconds of each step over `iters` runs (hipEvents on the stream). */
int32_t ku_hip_plan_time_steps(KuHipPlan *p, int32_t iters, double *out_ms, size_t cap);
/* Average GPU milliseconds of a whole plan launch over `iters` runs. */
double ku_hip_plan_time(KuHipPlan *p, int32_t iters, uint32_t use_graph);
/* Average GPU milliseconds of one round that launches each of `n` plans (one backend) once,
 * in order, over `iters` rounds: rotating independent input sets through the same kernels. */
double ku_hip_plans_time(KuHipPlan *const *plans, size_t n, int32_t iters, uint32_t use_graph);
void ku_hip_plan_free(KuHipPlan *p);

/* Generated HIP source of every fused region kernel for `roots`, concatenated and
 * separated by a line "// ----"; works without a GPU (hipRTC compiles each for gfx950 when
 * compile != 0). Returns the byte length; copies at most cap bytes into out. */
size_t ku_hip_codegen(KuGraph *g, const KuNode *roots, size_t n, uint32_t compile, uint8_t *out, size_t cap);

/* The e4m3 linear layer on caller-owned device buffers, the graph ku_amp_fp8 emits for one
 * layer as one call: sx = max|x| / 448 (computed on the device), xq = e4m3(x / sx) and
 * y = (xq @ wq^T) * sx * sw[n] rounded to y_dtype, on the fp8 MFMA GEMM. An all-zero x
 * (sx = 0) is divided by 1 instead, so y = 0 (not NaN).
 *   x  [m, k] KU_BF16 / KU_F16 / KU_F32, wq [n, k] KU_F8E4M3 (e.g. rows quantised with per-row
 *   absmax / 448 scales sw [n] f32), y [m, n] KU_BF16 / KU_F16 / KU_F32; all row-major, 16-byte
 *   aligned device pointers; k a multiple of 128.
 * Enqueued on `stream` (a hipStream_t; NULL = the backend's stream), asynchronously. Scratch (the
 * quantised activation, m*k bytes) is a workspace of the backend that grows on demand, so calls
 * on one backend must be ordered on one stream. Returns 0, or -1 with ku_last_error. */
int32_t ku_hip_linear_e4m3(const KuBackend *b, const void *x, uint32_t x_dtype, const uint8_t *wq, const float *sw,
                           void *y, uint32_t y_dtype, size_t m, size_t n, size_t k, void *stream);

/* ku_hip_linear_e4m3 without any allocation. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The scratch (absmax partials, sx, the quantised activation)
 * is a static device array of 16 MiB + 4352 bytes per GPU, held until the process ends, so
 * m * k <= 16 MiB (larger sizes return -1 with an error). Runs on the current device and on
 * `stream` (NULL = the null stream); every call on one GPU shares that GPU's scratch, so calls
 * that overlap on one GPU race. Returns 0, or -1 with ku_last_error. */
int32_t ku_hip_linear_e4m3_noalloc(const void *x, uint32_t x_dtype, const uint8_t *wq, const float *sw, void *y,
                                   uint32_t y_dtype, size_t m, size_t n, size_t k, void *stream);

/* Counters of a backend into out[0..cap): launches per kind (fused, gemm, attention, upload,
 * download), then plans built, constants uploaded and constants cached (plans and constants
 * are cached by graph content, so an equal graph rebuilt per call adds to neither); returns
 * the number of evals. */
uint64_t ku_hip_profile(const KuBackend *b, uint64_t *out_launches, size_t cap);

/* ---- collision-free entry set ----
 *
 * No counterpart in the reference. kurumi's own library (rlib, cdylib and staticlib of the
 * `kurumi` crate, kurumi/Cargo.toml:12-13) exports the same unprefixed ku_* names as this one,
 * so a process holding both (kurumi's CPU backend and C ABI plus this HIP backend) cannot reach
 * this library through those names: the dynamic linker binds each name to whichever definition
 * it finds first. ku_hip_api is the one name such a process binds; the table it returns points
 * at this library's own definitions, and the library binds its internal calls to itself
 * (linked with -Bsymbolic-functions), so every call through the table stays in
 * libkurumi_hip.so whatever else the process exports. The table covers the backend seam: errors,
 * backends, graphs, KGPH v2 decode, eval, plans, feeds, tensors and inspection; graphs are built
 * with kurumi's builders and handed over as KGPH v2 bytes.
 *
 * ku_hip_api(KU_HIP_API_VERSION) returns the table, or NULL (and ku_last_error) for a version
 * this library does not provide. Fields are only ever appended; `size` is sizeof the table the
 * library was built with. */
#define KU_HIP_API_VERSION 1u

typedef struct KuHipApi {
  uint32_t version; /* KU_HIP_API_VERSION */
  uint32_t size;    /* sizeof(KuHipApi) */
  const char *(*last_error)(void);
  KuBackend *(*backend_new)(uint32_t kind);
  void (*backend_free)(KuBackend *b);
  KuGraph *(*graph_new)(void);
  void (*graph_free)(KuGraph *g);
  KuRunnable *(*graph_deserialize)(const uint8_t *bytes, size_t len);
  KuGraph *(*runnable_take_graph)(KuRunnable *h);
  size_t (*runnable_output_count)(const KuRunnable *h);
  KuNode (*runnable_output)(const KuRunnable *h, size_t i);
  size_t (*runnable_input_count)(const KuRunnable *h);
  KuNode (*runnable_input_node)(const KuRunnable *h, size_t i);
  size_t (*runnable_input_name)(const KuRunnable *h, size_t i, uint8_t *out, size_t cap);
  void (*runnable_free)(KuRunnable *h);
  KuTensor *(*eval)(KuGraph *g, KuNode node, const KuBackend *backend);
  KuTensor *(*eval_with)(KuGraph *g, KuNode node, const KuBackend *backend, const KuFeeds *feeds);
  int32_t (*eval_many)(KuGraph *g, const KuNode *ids, size_t n, const KuBackend *backend, const KuFeeds *feeds,
                       KuTensor **out);
  KuPlan *(*plan_compile_on)(const KuBackend *b, const KuGraph *g, KuNode node);
  KuTensor *(*plan_run)(const KuPlan *p, const KuGraph *g, const KuFeeds *feeds);
  void (*plan_free)(KuPlan *p);
  KuFeeds *(*feeds_new)(void);
  void (*feeds_free)(KuFeeds *f);
  void (*feeds_set)(KuFeeds *f, KuNode node, const KuTensor *tensor);
  KuTensor *(*tensor_new)(uint32_t dtype, const uint8_t *data, size_t nbytes, const size_t *shape, size_t rank);
  void (*tensor_free)(KuTensor *t);
  size_t (*tensor_rank)(const KuTensor *t);
  void (*tensor_shape)(const KuTensor *t, size_t *out);
  uint32_t (*tensor_dtype)(const KuTensor *t);
  size_t (*tensor_nbytes)(const KuTensor *t);
  void (*tensor_bytes)(const KuTensor *t, uint8_t *out);
  size_t (*node_count)(const KuGraph *g, KuNode root);
  size_t (*dump)(const KuGraph *g, KuNode root, uint8_t *out, size_t cap);
} KuHipApi;

const KuHipApi *ku_hip_api(uint32_t version);

#ifdef __cplusplus
}
#endif
#endif /* KURUMI_HIP_H */
