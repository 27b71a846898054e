/*
 * A C11 caller of libmixmoe through include/mixmoe.h alone: the call
 * sequence the cgo executor performs (mxm_init, mxm_moe_create with the op's
 * IntParams / FloatParams and input count, mxm_moe_set_input per
 * Op.Inputs[1..], a forward), run on the reference's known-answer case,
 * TestMoEFeedForwardMatchesCPUOracle (gpu/moe_feed_forward_test.go:14-82):
 * B=1, T=4, D=3, E=3, FFN=4, swiglu, top-k 1 and 2, inputs from
 * patternedFloats (gpu/hgrn2_mlstm_scan_test.go:288-294).
 *
 * For each top-k it runs the host-buffer forward and the device-pointer
 * forward (mxm_malloc, mxm_memcpy_h2d, mxm_moe_forward, mxm_moe_synchronize,
 * mxm_memcpy_d2h), reads the routing back, and prints one JSON object per
 * line: {"top_k", "delta", "aux", "entropy", "delta_device_equal",
 * "top_idx", "counts", "rc_bad_shape", "rc_bad_rows", "rc_bad_handle"}.
 * The caller (tests/test_c_abi.py) compares them with the float64 fixtures
 * of the case.  Exit status 0 when every call returned what it should.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "mixmoe.h"

enum { B = 1, T = 4, D = 3, E = 3, FFN = 4, N = B * T };

/* gpu/hgrn2_mlstm_scan_test.go:288-294 */
static void patterned_floats(float* out, int n, double scale) {
  for (int i = 0; i < n; ++i)
    out[i] = (float)(scale * (sin((double)(i + 1)) * 0.7 + cos((double)((i + 3) % 11)) * 0.3));
}

static int report(const char* what, int rc) {
  char msg[512];
  mxm_last_error(msg, (int)sizeof msg);
  fprintf(stderr, "%s failed: rc=%d: %s\n", what, rc, msg);
  return 1;
}

static void print_floats(const char* key, const float* v, int n) {
  printf("\"%s\": [", key);
  for (int i = 0; i < n; ++i) printf("%s%.9g", i ? ", " : "", (double)v[i]);
  printf("]");
}

static void print_ints(const char* key, const int32_t* v, int n) {
  printf("\"%s\": [", key);
  for (int i = 0; i < n; ++i) printf("%s%d", i ? ", " : "", (int)v[i]);
  printf("]");
}

static int run_case(int top_k) {
  float x[N * D], router[D * E], w[E][3][D * FFN];
  patterned_floats(x, N * D, 0.17);
  patterned_floats(router, D * E, 0.23);
  for (int e = 0; e < E; ++e) {
    patterned_floats(w[e][0], D * FFN, 0.09 + e * 0.03);  /* w_gate [D, FFN] */
    patterned_floats(w[e][1], D * FFN, 0.11 + e * 0.03);  /* w_up   [D, FFN] */
    patterned_floats(w[e][2], FFN * D, 0.13 + e * 0.03);  /* w_down [FFN, D] */
  }
  /* prog.MoEFeedForward(inputs, ..., B, T, D, E, topK, 0, FFN, 0, 0) */
  const int32_t int_params[8] = {B, T, D, E, top_k, 0, FFN, 0};
  const float float_params[1] = {0.0f};
  const int n_inputs = 2 + 3 * E;
  int64_t op = mxm_moe_create(float_params, 1, int_params, 8, n_inputs, MXM_DTYPE_F32, 0);
  if (op == 0) return report("mxm_moe_create", 0);

  int fails = 0, rc;
  const int64_t shape_router[2] = {D, E}, shape_in[2] = {D, FFN}, shape_down[2] = {FFN, D};
  if ((rc = mxm_moe_set_input(op, 1, MXM_DTYPE_F32, shape_router, 2, router, 0)) != MXM_OK)
    fails += report("mxm_moe_set_input(router_w)", rc);
  for (int e = 0; e < E; ++e)
    for (int j = 0; j < 3; ++j) {
      const int64_t* shp = j == 2 ? shape_down : shape_in;
      if ((rc = mxm_moe_set_input(op, 2 + 3 * e + j, MXM_DTYPE_F32, shp, 2, w[e][j], 0)) != MXM_OK)
        fails += report("mxm_moe_set_input(expert)", rc);
    }
  /* argument errors are MXM_ERR_ARGS, a dead handle MXM_ERR_OP */
  const int rc_bad_shape = mxm_moe_set_input(op, 1, MXM_DTYPE_F32, shape_in, 2, router, 0);
  float delta[N * D], delta_dev[N * D], aux = 0.0f, ent = 0.0f;
  const int rc_bad_rows = mxm_moe_forward_host(op, x, MXM_DTYPE_F32, N + 1, delta, &aux, &ent);

  if ((rc = mxm_moe_forward_host(op, x, MXM_DTYPE_F32, N, delta, &aux, &ent)) != MXM_OK)
    fails += report("mxm_moe_forward_host", rc);
  int32_t top_idx[N * 2], counts[E];
  if ((rc = mxm_moe_routing(op, top_idx, NULL, counts, NULL, NULL, 1)) != MXM_OK)
    fails += report("mxm_moe_routing", rc);

  /* the same forward on device pointers */
  void *dx = NULL, *dd = NULL, *daux = NULL;
  if ((rc = mxm_malloc(&dx, (int64_t)sizeof x)) != MXM_OK) fails += report("mxm_malloc", rc);
  if ((rc = mxm_malloc(&dd, (int64_t)sizeof delta)) != MXM_OK) fails += report("mxm_malloc", rc);
  if ((rc = mxm_malloc(&daux, 8)) != MXM_OK) fails += report("mxm_malloc", rc);
  int device_equal = 0;
  if (!fails) {
    float aux_dev[2];
    if ((rc = mxm_memcpy_h2d(dx, x, (int64_t)sizeof x)) != MXM_OK) fails += report("h2d", rc);
    if ((rc = mxm_moe_forward(op, dx, MXM_DTYPE_F32, N, (float*)dd, (float*)daux,
                              (float*)daux + 1)) != MXM_OK)
      fails += report("mxm_moe_forward", rc);
    if ((rc = mxm_moe_synchronize(op)) != MXM_OK) fails += report("mxm_moe_synchronize", rc);
    if ((rc = mxm_memcpy_d2h(delta_dev, dd, (int64_t)sizeof delta_dev)) != MXM_OK)
      fails += report("d2h", rc);
    if ((rc = mxm_memcpy_d2h(aux_dev, daux, 8)) != MXM_OK) fails += report("d2h", rc);
    device_equal = !fails && memcmp(delta, delta_dev, sizeof delta) == 0 &&
                   memcmp(&aux, &aux_dev[0], 4) == 0 && memcmp(&ent, &aux_dev[1], 4) == 0;
  }
  mxm_free(dx);
  mxm_free(dd);
  mxm_free(daux);
  if ((rc = mxm_moe_destroy(op)) != MXM_OK) fails += report("mxm_moe_destroy", rc);
  const int rc_bad_handle = mxm_moe_synchronize(op);

  printf("{\"top_k\": %d, ", top_k);
  print_floats("delta", delta, N * D);
  printf(", \"aux\": %.9g, \"entropy\": %.9g, \"delta_device_equal\": %s, ", (double)aux,
         (double)ent, device_equal ? "true" : "false");
  print_ints("top_idx", top_idx, N * top_k);
  printf(", ");
  print_ints("counts", counts, E);
  printf(", \"rc_bad_shape\": %d, \"rc_bad_rows\": %d, \"rc_bad_handle\": %d}\n", rc_bad_shape,
         rc_bad_rows, rc_bad_handle);
  fflush(stdout);
  if (rc_bad_shape != MXM_ERR_ARGS || rc_bad_rows != MXM_ERR_ARGS || rc_bad_handle != MXM_ERR_OP)
    ++fails;
  return fails;
}

int main(void) {
  int rc = mxm_init();
  if (rc != MXM_OK) return report("mxm_init", rc);
  printf("{\"device\": \"%s\"}\n", mxm_device_name());
  int fails = 0;
  for (int top_k = 1; top_k <= 2; ++top_k) fails += run_case(top_k);
  return fails ? 1 : 0;
}
