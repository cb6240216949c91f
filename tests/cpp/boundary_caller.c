/* A plain C caller of the drop-in boundary: every header of include/ must
 * compile as C (the extern "C" view an FFI binding sees), and the host-only
 * entry points must link and agree with the reference's formulas
 * (src/gemma4_kv_cache.cuh:28-38, src/gemma4_kv_cache.cu:76-105). Built and
 * run by tests/test_cpp_boundary.py. */
#include "gemma4_attention_output.h"
#include "gemma4_flash_attention.h"
#include "gemma4_kv_cache.h"
#include "gemma4_runtime.h"

#include <stdio.h>

int main(void) {
  const Gemma4KvCacheConfig c = gemma4_kv_cache_make_config(false, 64, 16, 65);
  const long long off = (long long)gemma4_kv_cache_offset(&c, 1, 2, 3, 4, 5);
  const long long expect = ((((1LL * 64 + 2) * 16 + 3) * 8 + 4) * 256 + 5);
  int32_t table[4] = {-1, -1, -1, -1}, slots[4] = {-1, -1, -1, -1};
  Gemma4KvCacheConfig r = gemma4_kv_cache_make_config(false, 4, 2, 4);
  r.batch_size = 1;
  const int ok = off == expect && gemma4_kv_cache_layer_index(5, true) == 0 &&
                 gemma4_kv_cache_layer_index(5, false) == -1 &&
                 gemma4_kv_cache_ensure_page_ptr(table, slots, 4, &r, 0, 7) == 3 &&
                 slots[3] == 3 && table[0] == -1;
  printf(ok ? "c caller ok\n" : "c caller FAILED\n");
  return ok ? 0 : 1;
}
