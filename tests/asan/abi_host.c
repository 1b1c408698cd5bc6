/* Host-side paths of the C ABI without a GPU, built with AddressSanitizer and UndefinedBehaviorSanitizer
 * (tests/test_asan_host.py): config validation, argument checks, forged and NULL handles, the no-device error.
 * Exits 0 when every call returns the documented status; the sanitizers abort on a memory or UB error. */
#include <stdio.h>
#include <string.h>

#include "ha.h"

static int fails = 0;
#define EXPECT(call, want)                                                                                   \
  do {                                                                                                       \
    int rc_ = (call);                                                                                        \
    if (rc_ != (want)) {                                                                                     \
      fprintf(stderr, "%s: got %d, want %d (%s)\n", #call, rc_, (int)(want), ha_last_error());               \
      fails++;                                                                                               \
    }                                                                                                        \
  } while (0)

int main(void) {
  unsigned char kinds[4] = {HA_LINEAR_ATTENTION, HA_LINEAR_ATTENTION, HA_LINEAR_ATTENTION, HA_FULL_ATTENTION};
  ha_config c;
  memset(&c, 0, sizeof c);
  c.n_layers = 4; c.layer_kind = kinds; c.batch = 2; c.max_ctx = 4096;
  c.H = 16; c.DK = 128; c.DV = 128; c.conv_k = 4; c.lin_stride = 8256; c.lin_dtype = HA_F32; c.lin_gnorm = 1;
  c.HQ = 8; c.HK = 2; c.HD = 256; c.rot_dim = 64; c.full_stride = 5120; c.full_dtype = HA_F16;
  c.rope_theta = 1e7f; c.eps = 1e-6f;
  ha_engine* e = NULL;
  ha_config bad = c;
  bad.DK = 64;
  EXPECT(ha_create(&bad, 0, &e), HA_ERR_ARG);
  bad = c; bad.eps = 1e-5f;
  EXPECT(ha_create(&bad, 0, &e), HA_ERR_ARG);
  bad = c; kinds[1] = 9;
  EXPECT(ha_create(&bad, 0, &e), HA_ERR_ARG);
  kinds[1] = HA_LINEAR_ATTENTION;
  EXPECT(ha_create(NULL, 0, &e), HA_ERR_ARG);
  EXPECT(ha_create(&c, 0, NULL), HA_ERR_ARG);
  EXPECT(ha_create(&c, 0, &e), HA_ERR_DEVICE); /* no GPU in this process */

  unsigned int forged[64];
  memset(forged, 0, sizeof forged);
  const unsigned int magics[3] = {0x48415350u, 0x48414D4Eu, 0x4841454Eu};
  int P = 0;
  for (int i = 0; i < 3; i++) {
    forged[0] = magics[i];
    void* h = forged;
    EXPECT(ha_snapshot_tokens((const ha_snapshot*)h, &P), HA_ERR_HANDLE);
    EXPECT(ha_snapshot_layout((const ha_snapshot*)h, &P, &P), HA_ERR_HANDLE);
    EXPECT(ha_snapshot_read((const ha_snapshot*)h, 0, "state", forged, 4), HA_ERR_HANDLE);
    EXPECT(ha_snapshot_release((ha_snapshot*)h), HA_ERR_HANDLE);
    EXPECT(ha_snapshot_destroy((ha_snapshot*)h), HA_ERR_HANDLE);
    EXPECT(ha_destroy((ha_engine*)h), HA_ERR_HANDLE);
    EXPECT(ha_forward((ha_engine*)h, 1, NULL, NULL, NULL, NULL, NULL), HA_ERR_HANDLE);
    EXPECT(ha_mnb_forward((ha_mnb*)h, 1, h, h, NULL), HA_ERR_HANDLE);
    EXPECT(ha_mnb_forward_noalloc((ha_mnb*)h, 1, h, h, NULL), HA_ERR_HANDLE);
    EXPECT(ha_mnb_destroy((ha_mnb*)h), HA_ERR_HANDLE);
    EXPECT(ha_embed((const ha_mnb*)h, 1, h, h, NULL), HA_ERR_HANDLE);
  }
  EXPECT(ha_snapshot_tokens(NULL, &P), HA_ERR_HANDLE);
  EXPECT(ha_destroy(NULL), HA_ERR_HANDLE);
  EXPECT(ha_mnb_destroy(NULL), HA_OK);
  ha_mnb_format f = {5, 32, 0};
  ha_mnb* w = NULL;
  EXPECT(ha_mnb_create(16, 2048, &f, forged, forged, NULL, 0, &w), HA_ERR_ARG);
  f.bits = 4;
  EXPECT(ha_mnb_create(16, 2048, &f, forged, forged, NULL, 0, &w), HA_ERR_DEVICE);
  EXPECT(ha_fwht(NULL, 0, 16, 0, NULL), HA_ERR_ARG);
  EXPECT(ha_add_norm(1, 12, 1, forged, NULL, (const float*)forged, forged, 0, NULL, 1e-6f, 0, NULL), HA_ERR_ARG);
  EXPECT(ha_silu_mul(1, 7, forged, forged, 0, NULL), HA_ERR_ARG);
  EXPECT(ha_add_bias(0, 8, forged, (const float*)forged, 0, NULL), HA_ERR_ARG);
  if (ha_abi_version() != HA_ABI_VERSION) fails++;
  printf("abi_host: %d failures\n", fails);
  return fails ? 1 : 0;
}
