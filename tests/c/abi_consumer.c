/* A plain C caller of the library, built against include/flowedge.h and linked with
 * -lflowedge_amd: the GPU-free part of the ABI (argument validation, thread-local error text,
 * the weights store and the model digest). Prints "ok <digest hex>" and exits 0 on success. */
#include <stdio.h>
#include <string.h>

#include "flowedge.h"

static int fail(const char* what) {
  fprintf(stderr, "FAIL %s (last error: \"%s\")\n", what, fe_engine_last_error());
  return 1;
}

int main(int argc, char** argv) {
  float buf[4] = {0};
  size_t remaining = 77;
  fe_condition_metadata md;
  fe_action_metadata amd;
  fe_model_digest digest;
  fe_weights* w;
  int i;
  if (argc != 2) return fail("usage: abi_consumer <checkpoint.safetensors>");
  if (fe_engine_last_error() == NULL) return fail("last_error is never NULL");
  if (fe_engine_sample_diffusion(NULL, buf, buf, 10, FE_DIFFUSION_DDIM, 0, buf) !=
      FE_STATUS_INVALID_ARGUMENT)
    return fail("sample_diffusion(NULL)");
  if (strstr(fe_engine_last_error(), "Invalid arguments") == NULL) return fail("error text");
  if (fe_engine_flow_advance(NULL, 1, buf, &remaining) != FE_STATUS_INVALID_ARGUMENT ||
      remaining != 77)
    return fail("flow_advance(NULL)");
  if (fe_engine_make_condition_metadata(NULL, 0, 0, 0, 1, FE_SOLVER_EULER, &md) !=
      FE_STATUS_INVALID_ARGUMENT)
    return fail("make_condition_metadata(NULL)");
  if (fe_engine_flow_action_metadata(NULL, &amd) != FE_STATUS_INVALID_ARGUMENT)
    return fail("flow_action_metadata(NULL)");
  fe_engine_cancel_before(NULL, 3);
  fe_engine_free(NULL);
  if (fe_engine_load(NULL) != NULL) return fail("load(NULL)");
  w = fe_weights_load(argv[1]);
  if (w == NULL) return fail("weights_load");
  if (fe_weights_size_bytes(w) == 0) return fail("weights_size_bytes");
  if (fe_weights_model_digest(w, &digest) != FE_STATUS_OK) return fail("weights_model_digest");
  fe_weights_free(w);
  printf("ok ");
  for (i = 0; i < FE_MODEL_DIGEST_BYTES; ++i) printf("%02x", digest.bytes[i]);
  printf("\n");
  return 0;
}
