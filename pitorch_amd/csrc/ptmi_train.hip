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

}  // extern "C"
