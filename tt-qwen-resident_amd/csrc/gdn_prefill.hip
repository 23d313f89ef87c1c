// Chunked-prefill gated delta rule (WY/UT form) on gfx950.
#include "qs_common.h"

extern "C" size_t qs_gdn_chunk_prefill_workspace_bytes(int T, int NK, int NV, int DK, int DV, int chunk) {
    (void)T, (void)NK, (void)NV, (void)DK, (void)DV, (void)chunk;
    return 256;
}

extern "C" int qs_gdn_chunk_prefill(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *g,
                                    const float *beta, const float *initial_state, uint16_t *o, float *final_state,
                                    void *workspace, int T, int NK, int NV, int DK, int DV, int chunk, float scale,
                                    float eps, void *stream) {
    (void)q, (void)k, (void)v, (void)g, (void)beta, (void)initial_state, (void)o, (void)final_state;
    (void)workspace, (void)T, (void)NK, (void)NV, (void)DK, (void)DV, (void)chunk, (void)scale, (void)eps;
    (void)stream;
    QS_REQUIRE(false, "qs_gdn_chunk_prefill: not built yet");
}
