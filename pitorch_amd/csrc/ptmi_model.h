// Device-resident model state shared by the decode and training units.
#pragma once

#include "ptmi_internal.h"

#include <vector>

namespace ptmi {

// Per-step control block in device memory.  Kernels of a captured decode
// step read the position and input token from here, so one graph serves
// every position.
struct DecodeCtl {
    int tok_in;      // token fed at `pos`
    int pos;         // current position
    int n_prompt;    // generate: positions < n_prompt-1 force prompt[pos+1]
    int next;        // argmax of the last step's logits
    // The host writes only the four fields above.
    int seq;         // steps run by the one-kernel decode step (its tags are seq + 1)
    int err;         // nonzero: a wait of the one-kernel step timed out
};

struct TrainState;   // defined by the training unit

constexpr int kMaxHeadDim = 128;
constexpr int kMaxSeqLen = 4096;    // 8 attention chunks of <= 512 positions

}  // namespace ptmi

struct ptmi_model {
    ptmi::Resident *res = nullptr;
    ptmi::Config c{};
    int max_T = 0;
    int host_pos = 0;
    // decode buffers (device)
    float *mem = nullptr;
    float *x = nullptr, *xb = nullptr, *q = nullptr, *hb = nullptr, *logits = nullptr;
    float *kc = nullptr, *vc = nullptr;
    float *part_o = nullptr, *part_ml = nullptr;   // attention chunk partials
    int attn_chunk = 0, attn_chunks = 0;
    ptmi::DecodeCtl *ctl = nullptr;
    int *prompt = nullptr, *out_tokens = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    // A second graph of graph_steps consecutive steps (PTMI_DECODE_GRAPH_STEPS,
    // 1 = none), launched while at least that many steps remain
    int graph_steps = 8;
    hipGraph_t graph_k = nullptr;
    hipGraphExec_t exec_k = nullptr;
    bool eager = false;                  // PTMI_DECODE_EAGER=1: no graph
    bool prefetch = true;                // PTMI_NO_PREFETCH=1: no L2 prefetch blocks
    // Which weights each launch of the step prefetches (into the MALL,
    // where they outlive the kernel boundary), one letter per producer:
    // QKV, attention, Wo, w1|w3, w2, classifier, argmax.  Targets, relative
    // to the producer's layer l: o = Wo_l, f = w1|w3_l, d = w2_l,
    // q = QKV_{l+1} (the next token's layer 0 after the last layer), O = Wo_{l+1},
    // F = w1|w3_{l+1}, '-' = none.  PTMI_PREFETCH_PLAN overrides it.
    char prefetch_plan[8] = "ofd---q";
    float *sink = nullptr;               // prefetch load sink
    // one-kernel decode step (null step_mem: the multi-kernel step)
    uint64_t *step_mem = nullptr;        // its tagged exchange buffers
    void *step_args = nullptr;           // its argument block (device memory)
    int step_nb = 0;                     // its workgroups (matvec and attention)
    const void *step_fn = nullptr;       // its kernel
    int step_plan = -1;                  // why it runs or not (plan_step: 0 runs, 1 shape, 2 residency)
    int step_chunk = 0, step_chunks = 0; // attention positions per unit, units per head
    uint64_t *step_stamps = nullptr;     // stage stamps (PTMI_STEP_STAMPS=1)
    int step_n_stamps = 0;
    std::vector<int> step_cuts;          // launch windows: stages [cuts[w], cuts[w+1])
    ptmi::TrainState *train = nullptr;
};

namespace ptmi {
int  train_create(ptmi_model *m);
void train_destroy(ptmi_model *m);
// 1/pt_sqrtf(head_dim) evaluated on the host (llama2.c:137)
float host_att_scale(int head_dim);
// The one-kernel decode step: set up (when PTMI_DECODE_STEP=1 and the shape
// has an instantiated kernel), tear down, enqueue one step.
int  decode_step_create(ptmi_model *m);
void decode_step_destroy(ptmi_model *m);
int  decode_step_windows(const ptmi_model *m);
int  launch_decode_step(ptmi_model *m, int w, hipStream_t s, hipEvent_t e0, hipEvent_t e1);
}
