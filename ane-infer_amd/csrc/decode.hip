// decode.hip — model weights, per-sequence state and the captured decode step.
#include "common.h"

using namespace anehip;

extern "C" int anehip_model_setup(anehip_ctx *ctx, const anehip_model_desc *desc) {
    (void)desc;
    return set_error(ctx->err, ANEHIP_EUNSUPPORTED, "model decode step not built yet");
}

extern "C" void anehip_model_teardown(anehip_ctx *ctx) { (void)ctx; }
