/*
 * libptmi — MI355X (gfx950) projection hot path for pitorch-style LLaMA-2.
 *
 * A C-ABI shared library: plain pointers and sizes, no C++ or torch types.
 * Every entry point that can fail returns a ptmi status (0 = PTMI_OK) and
 * leaves a message in ptmi_last_error().  Entry points whose reference
 * counterpart returns void (the pt_matvec_fn drop-in) report failure the
 * way the reference does — a panic: message on stderr, then abort().
 *
 * Threading: one library state per process, bound to one GPU and one HIP
 * stream; calls are not re-entrant (the reference is single-threaded bare
 * metal, pitorch/pt.c:19, pitorch/runtime/arena.c:5-8).
 *
 * Reference paths are relative to masonwang025/pitorch.
 */
#ifndef PTMI_H
#define PTMI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    PTMI_OK = 0,
    PTMI_ERR_ARG = 1,        /* bad shape / pointer / size                */
    PTMI_ERR_OOM = 2,        /* device allocation failed                  */
    PTMI_ERR_HIP = 3,        /* HIP runtime error                         */
    PTMI_ERR_STATE = 4,      /* not initialised, or wrong object state    */
    PTMI_ERR_NODEV = 5       /* no GPU visible                            */
};

/* ── library lifetime ─────────────────────────────────────────────────
 * Replaces the VideoCore bring-up in pt_pi_init (pitorch/pt.c:38-44:
 * qpu_enable, perf_init, gpu_arena_init).  ptmi_init selects the device
 * and creates the library's stream; it is implied by every other entry
 * point (device 0) if not called first.                                */
int         ptmi_init(int device);
void        ptmi_shutdown(void);
const char *ptmi_last_error(void);
int         ptmi_last_status(void);
void       *ptmi_stream(void);          /* hipStream_t of all launches */
int         ptmi_sync(void);            /* wait for the stream         */

/* ── weight residency ─────────────────────────────────────────────────
 * Register a llama2.c .bin blob (header + tensors, pitorch/model/
 * llama2.c:9-70; size per pt_file_size, llama2.c:21-47).  The tensors are
 * copied once into HBM in the device layout (per layer [wq;wk;wv] and
 * row-interleaved [w1|w3]); afterwards any host pointer into the blob's
 * weight tensors passed to ptmi_matvec resolves to its device copy.
 * Replaces: the Pi's weights-in-ARM-RAM read through the TMU bus alias
 * (pitorch/ops/matvec/matvec.c:13-30).
 * Registrations are counted holds on one device copy per blob address:
 * each ptmi_register_weights call and each live ptmi_model over the blob
 * holds it, and the copy is freed when the last hold ends.  Registering a
 * blob whose size or 28-byte header differs from the registration still
 * held at that address fails with PTMI_ERR_STATE.                       */
int ptmi_register_weights(const void *blob, size_t bytes);
/* Re-upload [ptr, ptr+bytes) of a registered blob after host writes
 * (pitorch/train/pt_train.c:870-896 mutates W in place), or of a
 * registered buffer (below).                                            */
int ptmi_invalidate(const void *ptr, size_t bytes);
/* End one ptmi_register_weights hold.  Refused (PTMI_ERR_STATE) while a
 * model created over the blob is alive: destroy the models first.       */
int ptmi_unregister_weights(const void *blob);
/* Register a plain host buffer of floats that ptmi_matvec reads as W many
 * times between host writes, e.g. the backward's host-transposed weights
 * (w_transpose, pitorch/train/pt_train.c:405-407, filled by transpose()
 * at :588-594 and :662-679, then read by T-1 matvecs each).  It is copied
 * to HBM once; a W that lies inside it is served from that copy instead of
 * being uploaded per call (37 MB per call for the transposed classifier).
 * After the host rewrites part of it, ptmi_invalidate(ptr, bytes) over
 * that part re-uploads it; until then matvecs read the old contents.
 * Must not overlap a registered blob or buffer.  No reference counterpart:
 * the Pi reads host memory directly through the TMU.                    */
int ptmi_register_buffer(const void *p, size_t bytes);
int ptmi_unregister_buffer(const void *p);

/* ── matvec: y[out_dim] = W[out_dim, in_dim] . x[in_dim] ──────────────
 * ptmi_matvec has exactly the pt_matvec_fn signature
 * (pitorch/model/llama2.h:73-75) and replaces matvec_gpu/smatvec_tmu
 * (pitorch/pt.c:21-25, pitorch/ops/matvec/matvec.c:13-86).  Host pointers;
 * W is resolved through the residency map, else uploaded for the call.
 * y is fully overwritten.  Unlike smatvec_tmu there is no out_dim%16
 * constraint (matvec.c:15-16).  Panics (stderr + abort) on error, as the
 * reference's demand() does.                                           */
void ptmi_matvec(const float *W, const float *x, float *y, int out_dim, int in_dim);
/* Same, returning a status instead of panicking. */
int  ptmi_matvec_checked(const float *W, const float *x, float *y, int out_dim, int in_dim);
/* Device pointers, enqueued on `stream` (NULL = the library stream), no
 * synchronisation.  ld = row stride of W in floats (>= in_dim).        */
int  ptmi_matvec_dev(const float *dW, long ld, const float *dx, float *dy,
                     int out_dim, int in_dim, void *stream);
/* Ablation baseline, same arguments and result: the same kernel geometry,
 * but every row pass re-reads its slice of x from memory instead of
 * holding it in registers for the whole wave.  The counterpart of the
 * reference's smatvec_tmu_no_packing (pitorch/ops/matvec/
 * matvec_no_packing.c:1-10,25-85), which re-packs x for every dispatch
 * and is kept there as the baseline of that design choice.  Needs
 * in_dim % 4 == 0, in_dim <= 2304, 16-byte aligned rows.               */
int  ptmi_matvec_dev_xreread(const float *dW, long ld, const float *dx, float *dy,
                             int out_dim, int in_dim, void *stream);

/* ── training GEMMs (fp32, MFMA) ──────────────────────────────────────
 * C[M,N] (+)= A[M,K] . B[K,N], all row-major.  Replaces sgemm_rect_tmu
 * (pitorch/ops/gemm/gemm_rect.h:24-26; the num_qpus argument has no
 * meaning here and is dropped) and sgemm_cpu (gemm.h:19-20, accumulate=0).
 * Host pointers.                                                        */
int ptmi_sgemm_rect(const float *A, const float *B, float *C,
                    int M, int K, int N, int accumulate);
/* Exactly the signature of sgemm_rect_tmu (pitorch/ops/gemm/gemm_rect.h:
 * 24-26): num_qpus selects nothing (the matrix cores need no worker
 * count) but must lie in 1..12 as there (gemm_rect.c:34); no N%16
 * constraint (:33).  Panics (stderr + abort) on error, as the
 * reference's demand() does.                                            */
void ptmi_sgemm_rect_tmu(const float *A, const float *B, float *C,
                         int M, int K, int N, int num_qpus, int accumulate);
/* Exactly the signature of sgemm_cpu (pitorch/ops/gemm/gemm.h:19-20):
 * C[M,N] = A[M,K] . B[K,N] on the GPU.  Panics on error.               */
void ptmi_sgemm_cpu(const float *A, const float *B, float *C, int M, int K, int N);
/* dW[out,in] += sum_t dY[t,out] * X[t,in]  (TN GEMM, no host transpose).
 * Exactly the signature of matmul_backward_weight_batched
 * (pitorch/train/pt_train.c:475-477, void); T = 1 is the rank-1
 * matmul_backward_weight (pitorch/train/pt_backward_ops.c:43-49).
 * Host pointers.  Panics on error.                                      */
void ptmi_matmul_backward_weight_batched(float *d_W, const float *d_y_all,
                                         const float *x_all, int out_dim,
                                         int in_dim, int T);
/* Same, returning a status instead of panicking. */
int  ptmi_matmul_backward_weight_batched_checked(float *d_W, const float *d_y_all,
                                                 const float *x_all, int out_dim,
                                                 int in_dim, int T);
/* dX[T,in] (+)= dY[T,out] . W[out,in]  (NN GEMM).  The batched form of
 * backward_input_pretrans/matmul_backward_input (pt_train.c:442-453,
 * pt_backward_ops.c:32-41) without the host transpose.  Host pointers. */
int ptmi_matmul_backward_input_batched(float *d_x_all, const float *W,
                                       const float *d_y_all, int out_dim,
                                       int in_dim, int T, int accumulate);
/* Device-pointer forms.  op: 0 = NN  C(+)=A.B,      A[M,K]  B[K,N]
 *                            1 = TN  C(+)=A^T.B,    A[K,M]  B[K,N]
 *                            2 = NT  C(+)=A.B^T,    A[M,K]  B[N,K]
 * lda/ldb/ldc are row strides in floats.                                */
int ptmi_gemm_dev(int op, const float *dA, long lda, const float *dB, long ldb,
                  float *dC, long ldc, int M, int N, int K, int accumulate,
                  void *stream);
/* ptmi_gemm_dev without any allocation.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, same kernels and the same bits as ptmi_gemm_dev; its
 * split-K partial sums go to a fixed 16 MiB device scratch array that the
 * library holds on each GPU for the life of the process, located once by
 * ptmi_init (which must have been called: PTMI_ERR_STATE otherwise).  A
 * GEMM whose K split needs more than 4 Mi floats of partials (splits*M*N)
 * is rejected with PTMI_ERR_ARG before anything is enqueued.  Every call
 * on a GPU shares that GPU's scratch: calls that can overlap on one GPU
 * (other streams, other threads) race.  Nothing needs clearing between
 * calls: each launch writes every partial it later reads.              */
int ptmi_gemm_dev_noalloc(int op, const float *dA, long lda, const float *dB, long ldb,
                          float *dC, long ldc, int M, int N, int K, int accumulate,
                          void *stream);

/* ── device-resident model (decode + training) ────────────────────────
 * One registered blob plus device state: KV cache, activations and, when
 * max_T > 0, training buffers and gradients.  Replaces pt_host_init /
 * pt_pi_init (pitorch/pt.c:38-114, 232-248).                            */
typedef struct ptmi_model ptmi_model_t;
int  ptmi_model_create(const void *blob, size_t bytes, int max_T, ptmi_model_t **out);
void ptmi_model_destroy(ptmi_model_t *m);
int  ptmi_model_config(const ptmi_model_t *m, int cfg7[7]);
/* pt_reset_kv (pitorch/pt.c:273-280): zero the KV cache, pos = 0. */
int  ptmi_model_reset_kv(ptmi_model_t *m);
/* pt_forward_step (pitorch/pt.c:267-271): forward `token` at the current
 * position through one graph launch, pos += 1, *next = argmax(logits).  */
int  ptmi_model_forward_step(ptmi_model_t *m, int token, int *next);
/* Copy the last step's logits [vocab] to host memory. */
int  ptmi_model_logits(ptmi_model_t *m, float *out);
int  ptmi_model_pos(const ptmi_model_t *m);
/* Greedy pt_generate over token ids (pitorch/text/pt_text.c:314-361 with
 * temperature 0): zero the KV cache, force prompt[1..n_prompt-1] during
 * prefill, then argmax.  All steps run back to back on the device; the
 * host waits once.  out[i] = token chosen after position i;
 * *n_out = positions run (stops after a sampled 1 or 2 when stop_on_eos). */
int  ptmi_model_generate(ptmi_model_t *m, const int *prompt, int n_prompt,
                         int max_tokens, int stop_on_eos, int *out, int *n_out);
/* Enqueue `n_steps` greedy decode steps from the current position without
 * waiting (benchmark form of the loop above; tokens stay on the device).
 * Its errors are deferred: a wait of the one-kernel step that timed out
 * makes the rest of the submission do nothing, and is reported by the
 * next ptmi_model_sync (or forward_step / generate) on this model.      */
int  ptmi_model_decode_async(ptmi_model_t *m, int first_token, int n_steps);
/* Wait for the model's enqueued work; PTMI_ERR_STATE when a one-kernel
 * decode step of it timed out (the model stays usable afterwards).  No
 * counterpart in the reference (its steps are synchronous, pt.c:267-271). */
int  ptmi_model_sync(ptmi_model_t *m);
/* Kernel timing: run `n_steps` decode steps eagerly (no graph) with HIP
 * events around every launch, from the current position.  role_ms[i] is
 * the summed kernel time and role_launches[i] the launch count of role i:
 * 0 QKV matvec, 1 attention, 2 Wo matvec, 3 w1|w3 matvec, 4 w2 matvec,
 * 5 classifier matvec, 6 argmax; 7 the whole step when it runs as one
 * kernel (then the only role).  Takes the place of the reference's
 * per-matvec V3D counters (pitorch/profiler/profiler.h:6-28).           */
int  ptmi_model_profile(ptmi_model_t *m, int first_token, int n_steps,
                        float role_ms[8], int role_launches[8]);
/* Stage timing of the one-kernel decode step, for a model created with
 * PTMI_STEP_STAMPS=1 in the environment: for each of *n_wg workgroups,
 * *n_stamps = 1 + 10*n_layers + 4 readings of the GPU's 100 MHz real-time
 * counter taken by the LAST step: kernel start; per layer, the end of the
 * wait and the end of the work of QKV, attention, Wo, w1|w3, w2; then the
 * classifier's and the final argmax's.  0 where the workgroup had no
 * part in a stage.  out holds n_wg * n_stamps words, workgroup-major.   */
int  ptmi_model_step_stamps(ptmi_model_t *m, uint64_t *out, size_t n, int *n_stamps, int *n_wg);
/* Which decode step pt_forward_step (pitorch/pt.c:267-271) runs on.  The
 * one-kernel step needs a supported shape, one workgroup per compute unit
 * all resident at once (its workgroups wait for each other's results, so
 * one that cannot start would stall the others until their wait bound
 * runs out), and a workgroup of its own for every attention unit.  Pure
 * host arithmetic, no device call: cfg7 as ptmi_model_config, cus =
 * compute units, per_cu = workgroups of the step kernel one compute unit
 * holds at once (its occupancy).  *reason = 0 (one kernel: *grid
 * workgroups, *units of them attention units), 1 (shape not supported) or
 * 2 (grid or attention units do not fit): 1 and 2 take the multi-kernel
 * step.  Returns a status.  No counterpart in the reference (its decode
 * runs on one core).                                                    */
int  ptmi_decode_step_plan(const int cfg7[7], int cus, int per_cu, int *reason, int *grid, int *units);
/* The plan a model's creation took: as above, with the device's own
 * compute units and occupancy; -1 when PTMI_DECODE_STEP=0 forced the
 * multi-kernel step.                                                    */
int  ptmi_model_step_plan(const ptmi_model_t *m);
/* pt_train_step (pitorch/pt.c:339-364): zero grads, forward (loss),
 * backward, SGD on the device copy of the weights.                     */
int  ptmi_model_train_step(ptmi_model_t *m, const int *tokens, int T, float lr,
                           float *loss);
/* One device-timed span of a traced training step: the reference's trace
 * event (pitorch/profiler/trace.h:24-33, pt_trace_event_t) with times from
 * HIP events on the step's stream.  name/cat are static strings with the
 * reference's span tree (pt.c:339-364, pt_train.c:171-866): train_step,
 * zero_grads, forward, embedding, layer, qkv, attention, ffn, classifier,
 * loss, backward, cls_transpose, cls_weight_grad, transpose, wo, sgd,
 * plus weight_grads (the layers' weight gradients in one launch, which
 * the reference computes inside each layer's spans); layer = -1 outside
 * the layers; depth = nesting depth (train_step is 0).                  */
typedef struct {
    const char *name;
    const char *cat;        /* "train", "fwd", "bwd" */
    int         layer;
    int         depth;
    double      start_us;   /* from the beginning of train_step */
    double      dur_us;
} ptmi_span_t;
/* ptmi_model_train_step with HIP events around the phases (pt_train_step
 * with ctx->trace enabled, pt.c:339-364), enqueued without the graph
 * behind a short bounded busy kernel, so the step's kernels run back to
 * back and the spans time device work.  Spans are
 * written in the order they end, as trace.c records them; *n_spans gets
 * the step's span count, and a buffer of fewer than that many spans is an
 * error (nothing is written to it; the step has run).                  */
int  ptmi_model_train_step_trace(ptmi_model_t *m, const int *tokens, int T, float lr, float *loss,
                                 ptmi_span_t *spans, int max_spans, int *n_spans);
/* Copy the device weights back into a host blob of the same layout
 * (file order, pitorch/model/llama2.c:49-70).                           */
int  ptmi_model_read_weights(ptmi_model_t *m, void *blob, size_t bytes);
/* Copy the gradient buffer (pt_grads_t order, pitorch/train/
 * pt_train.c:342-370) of the last train step to host memory.           */
int  ptmi_model_read_grads(ptmi_model_t *m, float *out, size_t n_floats);

#ifdef __cplusplus
}
#endif
#endif
