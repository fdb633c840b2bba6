/* Links liboxide_paged_kv.a (no shared library) and calls its C ABI on paths that need
 * no GPU: argument errors of the reference's two kernel entry points, the host helpers
 * and the decode policy queries.  Prints "static link: N failures". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "oxide_paged_kv.h"
#include "oxide_workload.h"

static int failures = 0;
#define CHECK(c)                                             \
  do {                                                       \
    if (!(c)) {                                              \
      printf("FAILED %s:%d %s\n", __FILE__, __LINE__, #c);   \
      ++failures;                                            \
    }                                                        \
  } while (0)

int main(void) {
  /* reshape_and_cache with an unknown dtype code: the reference drops it silently,
   * this library records the error (crates/vllm-oxide/kernels/reshape_and_cache.cu:30-71). */
  oxide_clear_error();
  reshape_and_cache(NULL, NULL, NULL, NULL, NULL, 1, 8, 128, 7, NULL);
  CHECK(oxide_last_error() == OXIDE_ERR_UNSUPPORTED_DTYPE);
  CHECK(strcmp(oxide_error_string(OXIDE_ERR_UNSUPPORTED_DTYPE), "unsupported dtype code") == 0);
  oxide_clear_error();
  copy_blocks(NULL, NULL, NULL, 1, 256 * 8 * 128, OXIDE_DTYPE_BF16, NULL);
  CHECK(oxide_last_error() == OXIDE_ERR_INVALID_ARGUMENT);
  oxide_clear_error();
  /* Nothing to do: no error, no launch. */
  reshape_and_cache(NULL, NULL, NULL, NULL, NULL, 0, 8, 128, OXIDE_DTYPE_BF16, NULL);
  CHECK(oxide_last_error() == OXIDE_OK);

  CHECK(paged_decode_attention_workspace_size(64, 32, 8, 128, 8192) > 0);
  CHECK(paged_decode_attention_workspace_size(64, 32, 8, 128, 0) == 0);
  CHECK(paged_decode_attention_path_split_tokens(1, 64, 8, 8192) == 1024);

  float cs[4 * 128];
  CHECK(oxide_rope_cos_sin_cache(cs, 4, 128, 1000000.0f) == OXIDE_OK);
  CHECK(cs[0] == 1.0f && cs[64] == 0.0f);                   /* position 0: cos 1, sin 0 */
  CHECK(fabsf(cs[128] - cosf(1.0f)) < 1e-6f);               /* position 1, f_0 = 1 */

  uint16_t a[1001], b[1001];
  CHECK(oxide_fill_normal(a, 1001, 3, 4, OXIDE_DTYPE_BF16, 1) == 0);
  CHECK(oxide_fill_normal(b, 1001, 3, 4, OXIDE_DTYPE_BF16, 4) == 0);
  CHECK(memcmp(a, b, sizeof a) == 0);
  CHECK(oxide_fill_normal(a, 10, 0, 0, 9, 1) == 1);

  printf("static link: %d failures\n", failures);
  return failures != 0;
}
