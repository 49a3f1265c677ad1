// pkh_prefill.hip -- causal prefill on CDNA4 MFMA (placeholder until the kernel lands).
#include "pkh_internal.h"

namespace pkh {

bool prefill_supported(int head_dim, int group, int dtype) {
    (void)head_dim; (void)group; (void)dtype;
    return false;
}

int launch_prefill(const PrefillArgs& a, hipStream_t stream) {
    (void)a; (void)stream;
    return PKH_ERR_ARG;
}

}  // namespace pkh
