// Device-resident training step (pt_train_step, pitorch/pt.c:339-364).
#include "ptmi_model.h"

namespace ptmi {

struct TrainState {
    int dummy;
};

int train_create(ptmi_model *m) {
    (void)m;
    return set_error(PTMI_ERR_STATE, "device training step not available in this build");
}

void train_destroy(ptmi_model *m) {
    delete m->train;
    m->train = nullptr;
}

}  // namespace ptmi

using namespace ptmi;

extern "C" {

int ptmi_model_train_step(ptmi_model_t *m, const int *tokens, int T, float lr, float *loss) {
    (void)m; (void)tokens; (void)T; (void)lr; (void)loss;
    return set_error(PTMI_ERR_STATE, "device training step not available in this build");
}

int ptmi_model_read_grads(ptmi_model_t *m, float *out, size_t n_floats) {
    (void)m; (void)out; (void)n_floats;
    return set_error(PTMI_ERR_STATE, "device training step not available in this build");
}

int ptmi_sgemm_rect(const float *A, const float *B, float *C, int M, int K, int N, int accumulate) {
    (void)A; (void)B; (void)C; (void)M; (void)K; (void)N; (void)accumulate;
    return set_error(PTMI_ERR_STATE, "GEMM not available in this build");
}

int ptmi_matmul_backward_weight_batched(float *d_W, const float *d_y_all, const float *x_all, int out_dim,
                                        int in_dim, int T) {
    (void)d_W; (void)d_y_all; (void)x_all; (void)out_dim; (void)in_dim; (void)T;
    return set_error(PTMI_ERR_STATE, "GEMM not available in this build");
}

int ptmi_matmul_backward_input_batched(float *d_x_all, const float *W, const float *d_y_all, int out_dim,
                                       int in_dim, int T, int accumulate) {
    (void)d_x_all; (void)W; (void)d_y_all; (void)out_dim; (void)in_dim; (void)T; (void)accumulate;
    return set_error(PTMI_ERR_STATE, "GEMM not available in this build");
}

int ptmi_gemm_dev(int op, const float *dA, long lda, const float *dB, long ldb, float *dC, long ldc, int M, int N,
                  int K, int accumulate, void *stream) {
    (void)op; (void)dA; (void)lda; (void)dB; (void)ldb; (void)dC; (void)ldc; (void)M; (void)N; (void)K;
    (void)accumulate; (void)stream;
    return set_error(PTMI_ERR_STATE, "GEMM not available in this build");
}

}  // extern "C"
