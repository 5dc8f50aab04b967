/*
 * A plain C11 consumer of libvapi_kv.so through include/vapi_kv.h: the
 * header compiles as C and the host-side calls work without Python or a
 * GPU. Built and run by tests/test_abi.py (gcc). Each check names the
 * reference behaviour it follows; exit status 0 means every check held.
 */
#include <stdio.h>
#include <string.h>

#include "vapi_kv.h"

static int failures = 0;
#define CHECK(cond, what)                                         \
  do {                                                            \
    if (!(cond)) {                                                \
      ++failures;                                                 \
      fprintf(stderr, "FAIL %s (%s:%d)\n", what, __FILE__, __LINE__); \
    }                                                             \
  } while (0)

int main(void) {
  printf("%s\n", vapi_kv_version());

  /* block_bytes (backend.rs:695-708): config 4's 917,504-byte block, and a
   * chain with a K-only (Rows) pool adds its K alone. */
  vapi_kv_pool p;
  memset(&p, 0, sizeof p);
  p.k = (void*)16;
  p.v = (void*)32;
  p.layer_stride_bytes = 1u << 20;
  p.num_layers = 28;
  p.num_blocks = 8;
  p.block_size = 16;
  p.num_kv_heads = 4;
  p.head_dim = 128;
  p.dtype = VAPI_KV_BF16;
  p.layout = VAPI_KV_LAYOUT_HND;
  CHECK(vapi_kv_block_bytes(&p) == 917504, "block_bytes of config 4");
  vapi_kv_pool rows = p;
  rows.v = NULL;
  rows.num_layers = 1;
  rows.num_kv_heads = 1;
  rows.head_dim = 40;
  p.next = &rows;
  CHECK(vapi_kv_block_bytes(&p) == 917504 + 16 * 40 * 2, "block_bytes over a chain");

  /* pack_block_tables (attention.rs:414-430): [[0,1,2],[7]] -> [[0,1,2],[7,7,7]]. */
  const uint32_t offs[3] = {0, 3, 4}, data[4] = {0, 1, 2, 7};
  uint32_t packed[6] = {0};
  CHECK(vapi_pack_block_tables(2, offs, data, packed, 6) == 3, "pack width");
  const uint32_t want[6] = {0, 1, 2, 7, 7, 7};
  CHECK(memcmp(packed, want, sizeof want) == 0, "pack padding with the row's last block");
  CHECK(vapi_pack_block_tables(2, offs, data, packed, 5) < 0, "pack capacity check");

  /* ForwardBatch::validate (backend.rs:96-204): a 3-token prefill on 5
   * cached keys and a decode over 4-slot blocks; then a duplicate slot. */
  const uint32_t pos[4] = {5, 6, 7, 5}, slots[4] = {21, 22, 23, 1};
  const uint32_t cu_q[3] = {0, 3, 4}, cu_k[3] = {0, 8, 14};
  const uint32_t t_offs[3] = {0, 2, 4}, t_data[4] = {4, 5, 7, 0}, logits[2] = {2, 3};
  CHECK(vapi_forward_batch_validate(4, pos, slots, cu_q, cu_k, 2, t_offs, t_data, logits, 2, 8,
                                    4) == VAPI_KV_OK,
        "a valid batch");
  const uint32_t dup[4] = {21, 22, 23, 22};
  CHECK(vapi_forward_batch_validate(4, pos, dup, cu_q, cu_k, 2, t_offs, t_data, logits, 2, 8,
                                    4) == VAPI_KV_EINVAL,
        "a duplicate slot");
  CHECK(strstr(vapi_kv_last_error(), "slot 22") != NULL, "the reference's message");

  /* The spill store (spill.rs:225-241): host memory for two 10-byte blobs;
   * a third put drops the least recently used. */
  vapi_spill_store* s = NULL;
  CHECK(vapi_spill_open(NULL, 20, 0, &s) == VAPI_KV_OK && s, "spill open");
  uint8_t h[3][32];
  memset(h, 0, sizeof h);
  for (int i = 0; i < 3; ++i) h[i][0] = (uint8_t)(i + 1);
  uint8_t blob[10], got[16];
  memset(blob, 7, sizeof blob);
  CHECK(vapi_spill_put(s, h[0], blob, 10) == 0, "put 0");
  CHECK(vapi_spill_put(s, h[1], blob, 10) == 0, "put 1");
  CHECK(vapi_spill_get(s, h[0], got, sizeof got) == 10, "get 0");
  CHECK(vapi_spill_put(s, h[2], blob, 10) == 0, "put 2");
  CHECK(!vapi_spill_contains(s, h[1]), "least recently used dropped");
  CHECK(vapi_spill_contains(s, h[0]) && vapi_spill_contains(s, h[2]), "the rest held");
  CHECK(vapi_spill_get(s, h[1], got, sizeof got) == -1, "a miss");
  vapi_spill_stats st;
  vapi_spill_get_stats(s, &st);
  CHECK(st.ram_blocks == 2 && st.drops == 1 && st.hits == 1 && st.misses == 1, "stats");
  CHECK(vapi_spill_drain(s, 1) == 0, "nothing in flight");
  vapi_spill_close(s);

  /* Errors are codes and a message, never a crash. */
  CHECK(vapi_kv_append(NULL, 0, NULL, NULL, NULL, 1, NULL) == VAPI_KV_EINVAL, "null pool");
  CHECK(strlen(vapi_kv_last_error()) > 0, "an error message");

  printf("%s\n", failures ? "FAILED" : "all checks passed");
  return failures ? 1 : 0;
}
