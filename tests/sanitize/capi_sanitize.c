/* Host-side checks of the C ABI under AddressSanitizer and
 * UndefinedBehaviorSanitizer: descriptor validation, workspace sizing over
 * a grid of descriptors (every kernel family's size function), batch
 * sizing, the argument checks that return before any launch, and the status
 * strings.  No GPU work: every srw_forward / srw_backward call here is one
 * the library refuses on the host.  Built by tests/sanitize/Makefile; run by
 * tests/test_sanitize.py.  Exits non-zero on a wrong status; a sanitizer
 * finding aborts the program. */
#include <math.h>
#include <stdio.h>
#include <string.h>

#include "srw_amd.h"

static int failures = 0;
#define EXPECT(cond, ...)                         \
  do {                                            \
    if (!(cond)) {                                \
      fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      fprintf(stderr, __VA_ARGS__);               \
      fprintf(stderr, "\n");                      \
      ++failures;                                 \
    }                                             \
  } while (0)

static srw_desc_t make(int64_t T, int64_t D, int64_t dr, int64_t N, int R, int dtype, int gate, int stats,
                       uint32_t flags, int64_t chunk) {
  srw_desc_t d;
  srw_desc_init(&d);
  d.T = T;
  d.d_model = D;
  d.d_route = dr;
  d.n_units = N;
  d.n_routes = R;
  d.dtype = dtype;
  d.gate = gate;
  d.stats_mode = stats;
  d.flags = flags;
  d.chunk_size = chunk;
  return d;
}

int main(void) {
  EXPECT(srw_abi_version() == SRW_AMD_ABI_VERSION, "abi version");
  EXPECT(srw_desc_init(NULL) == SRW_EINVAL, "desc_init(NULL)");
  for (int s = -1; s <= 8; ++s) {
    const char* str = srw_status_string((srw_status_t)s);
    EXPECT(str != NULL && strncmp(str, "SRW_", 4) == 0, "status string %d", s);
  }

  /* workspace sizing over a grid: every family's sizing code on every shape */
  const int64_t Ts[] = {0, 1, 7, 64, 129, 4096};
  const int64_t Ds[] = {40, 64, 128, 384, 1024};
  const int64_t drs[] = {24, 32, 64, 128, 384, 1024};
  /* 4194304 / 8388608 units: the fp32 / bf16 tiled families' 32-bit tile
     offsets end there (256 rows x N64 x 4 or 2 bytes = 4 GiB); such shapes
     fall back to other families */
  const int64_t Ns[] = {1, 33, 100, 1580, 25200, 4194304, 8388608};
  const uint32_t flag_sets[] = {0, SRW_FLAG_DIAG, SRW_FLAG_EMULATE, SRW_FLAG_SPARSE_SKIP, SRW_FLAG_NO_FAST,
                                SRW_FLAG_POOL_CACHED, SRW_FLAG_TILED, SRW_FLAG_DIAG | SRW_FLAG_POOL_CACHED};
  long sized = 0, unsupported = 0;
  for (size_t a = 0; a < sizeof Ts / sizeof Ts[0]; ++a)
    for (size_t b = 0; b < sizeof Ds / sizeof Ds[0]; ++b)
      for (size_t c = 0; c < sizeof drs / sizeof drs[0]; ++c)
        for (size_t e = 0; e < sizeof Ns / sizeof Ns[0]; ++e)
          for (int R = 1; R <= 2; ++R)
            for (int dt = 0; dt <= 1; ++dt)
              for (int g = 0; g <= 1; ++g)
                for (int st = 0; st <= 2; ++st)
                  for (size_t f = 0; f < sizeof flag_sets / sizeof flag_sets[0]; ++f) {
                    const int dtype = dt ? SRW_F32 : SRW_BF16;
                    const int gate = g ? SRW_GATE_GELU_V401 : SRW_GATE_V41;
                    const int64_t chunk = (e + f) % 3 == 0 ? 0 : Ns[e] / 2;
                    srw_desc_t d = make(Ts[a], Ds[b], drs[c], Ns[e], R, dtype, gate, st, flag_sets[f], chunk);
                    size_t bytes = 12345;
                    const srw_status_t s = srw_workspace_size(&d, &bytes);
                    EXPECT(s == SRW_OK || s == SRW_EUNSUPPORTED, "workspace_size status %d", (int)s);
                    if (s == SRW_OK) {
                      ++sized;
                      EXPECT(Ts[a] != 0 || bytes == 0, "T = 0 sizes to 0 bytes, got %zu", bytes);
                      EXPECT(bytes % 256 == 0, "sizes are 256-byte multiples");
                    } else {
                      ++unsupported;
                    }
                    size_t bb = 0;
                    const srw_status_t sb = srw_backward_workspace_size(&d, &bb);
                    EXPECT(sb == SRW_OK || sb == SRW_EUNSUPPORTED, "backward size status %d", (int)sb);
                  }
  printf("sized %ld descriptors, %ld unsupported\n", sized, unsupported);
  EXPECT(sized > 1000, "most descriptors size");

  /* invalid descriptors: refused by sizing and by srw_forward alike */
  srw_tensors_t t;
  srw_outputs_t o;
  memset(&t, 0, sizeof t);
  memset(&o, 0, sizeof o);
  srw_desc_t bad[8];
  bad[0] = make(-1, 64, 64, 10, 1, SRW_BF16, SRW_GATE_V41, 0, 0, 0);
  bad[1] = make(4, 0, 64, 10, 1, SRW_BF16, SRW_GATE_V41, 0, 0, 0);
  bad[2] = make(4, 64, 64, 0, 1, SRW_BF16, SRW_GATE_V41, 0, 0, 0);
  bad[3] = make(4, 64, 64, 10, 3, SRW_BF16, SRW_GATE_V41, 0, 0, 0);
  bad[4] = make(4, 64, 64, 10, 1, 7, SRW_GATE_V41, 0, 0, 0);
  bad[5] = make(4, 64, 64, 10, 1, SRW_BF16, 9, 0, 0, 0);
  bad[6] = make(4, 64, 64, 10, 1, SRW_BF16, SRW_GATE_V41, 0, 0x100, 0);
  bad[7] = make(4, 64, 64, 10, 1, SRW_BF16, SRW_GATE_V41, 0, 0, -2);
  for (int i = 0; i < 8; ++i) {
    size_t bytes = 0;
    EXPECT(srw_workspace_size(&bad[i], &bytes) == SRW_EINVAL, "bad desc %d sizing", i);
    EXPECT(srw_forward(&bad[i], &t, &o, NULL, 0, NULL) == SRW_EINVAL, "bad desc %d forward", i);
    EXPECT(srw_forward_noalloc(&bad[i], &t, &o, NULL) == SRW_EINVAL, "bad desc %d noalloc", i);
  }
  srw_desc_t nan_desc = make(4, 64, 64, 10, 1, SRW_BF16, SRW_GATE_V41, 0, 0, 0);
  nan_desc.sharpness = NAN;
  size_t nb = 0;
  EXPECT(srw_workspace_size(&nan_desc, &nb) == SRW_EINVAL, "NaN sharpness");
  EXPECT(srw_workspace_size(NULL, &nb) == SRW_EINVAL, "NULL desc");

  /* argument checks before any launch */
  srw_desc_t d = make(16, 64, 32, 100, 1, SRW_BF16, SRW_GATE_V41, 0, 0, 0);
  EXPECT(srw_workspace_size(&d, NULL) == SRW_EINVAL, "NULL bytes");
  EXPECT(srw_forward(&d, NULL, NULL, NULL, 0, NULL) == SRW_EINVAL, "NULL tensors");
  EXPECT(srw_forward(&d, &t, &o, NULL, 0, NULL) == SRW_EINVAL, "null tensor pointers");
  srw_desc_t cached = d;
  cached.flags = SRW_FLAG_POOL_CACHED;
  EXPECT(srw_forward_noalloc(&cached, &t, &o, NULL) == SRW_EINVAL, "noalloc refuses pool-cached");
  srw_desc_t big = make(4096, 384, 384, 25200, 1, SRW_BF16, SRW_GATE_V41, 0, 0, 12600);
  EXPECT(srw_forward_noalloc(&big, &t, &o, NULL) == SRW_ESCRATCH, "noalloc scratch bound");
  srw_desc_t none = d;
  none.T = 0;
  EXPECT(srw_forward(&none, &t, &o, NULL, 0, NULL) == SRW_OK, "T = 0 is a no-op");

  /* batch sizing and checks */
  srw_desc_t ds[SRW_MAX_BATCH + 1];
  for (int i = 0; i <= SRW_MAX_BATCH; ++i) ds[i] = make(16 + i, 64, 32, 100 + 10 * i, 1, SRW_BF16, SRW_GATE_V41, 0, 0, 0);
  size_t total = 0, one = 0, sum = 0;
  EXPECT(srw_workspace_size_batch(SRW_MAX_BATCH, ds, &total) == SRW_OK, "batch sizing");
  for (int i = 0; i < SRW_MAX_BATCH; ++i) {
    srw_workspace_size(&ds[i], &one);
    sum += (one + 255) / 256 * 256;
  }
  EXPECT(total == sum, "batch size = aligned sum (%zu vs %zu)", total, sum);
  EXPECT(srw_workspace_size_batch(0, ds, &total) == SRW_EINVAL, "batch n = 0");
  EXPECT(srw_workspace_size_batch(SRW_MAX_BATCH + 1, ds, &total) == SRW_EINVAL, "batch n too large");
  srw_tensors_t ts[2];
  srw_outputs_t os[2];
  memset(ts, 0, sizeof ts);
  memset(os, 0, sizeof os);
  EXPECT(srw_forward_batch(2, ds, NULL, os, NULL, 0, NULL) == SRW_EINVAL, "batch NULL tensors");
  const srw_status_t sb = srw_forward_batch(2, ds, ts, os, NULL, 0, NULL);
  EXPECT(sb == SRW_EINVAL || sb == SRW_EWORKSPACE, "batch without workspace: %d", (int)sb);

  /* backward: argument checks */
  srw_cotangents_t ct;
  srw_grads_t gr;
  memset(&ct, 0, sizeof ct);
  memset(&gr, 0, sizeof gr);
  EXPECT(srw_backward(&d, &t, &ct, &gr, NULL, 0, NULL) == SRW_EINVAL || srw_backward(&d, &t, &ct, &gr, NULL, 0, NULL) == SRW_EUNSUPPORTED,
         "backward null pointers");
  EXPECT(srw_backward(NULL, &t, &ct, &gr, NULL, 0, NULL) == SRW_EINVAL, "backward NULL desc");

  const char* last = srw_last_path();
  EXPECT(last != NULL, "last path");
  EXPECT(srw_set_kernel_events(NULL, NULL) == SRW_OK, "clear kernel events");
  printf("%s: %d failures\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
