/* Random plan / plan_each / peek / note_token sequences against the slot
 * planner (locali_core.h, locali_planner.h), for a sanitizer build. */
#include <stdio.h>
#include <stdlib.h>
#include "locali_core.h"
#include "locali_planner.h"
static unsigned long long rng = 88172645463325252ull;
static unsigned r32(void) { rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17; return (unsigned)rng; }
int main(void) {
    for (int trial = 0; trial < 400; ++trial) {
        int keys_cap = 1 + r32() % 300, slots = 2 + r32() % 40;
        int prot = r32() % slots, policy = r32() % 2;
        locali_cache *c = locali_cache_create_policy(keys_cap, slots, prot, policy);
        if (!c) continue;
        for (int step = 0; step < 300; ++step) {
            int n = 1 + r32() % 12, m = r32() % 8;
            int32_t keys[12], pins[8];
            locali_cache_result res[12];
            for (int i = 0; i < n; ++i) keys[i] = (int32_t)(r32() % (keys_cap + 2)) - 1;   /* includes invalid */
            for (int i = 0; i < m; ++i) pins[i] = (int32_t)(r32() % (slots + 2)) - 1;
            int touch = r32() % 2;
            int rc = (r32() % 2) ? locali_cache_plan(c, keys, n, m ? pins : NULL, m, touch, res)
                                 : locali_cache_plan_each(c, keys, n, m ? pins : NULL, m, touch, res);
            (void)rc;
            if (r32() % 16 == 0) locali_cache_note_token(c);
            (void)locali_cache_peek(c, (int32_t)(r32() % (keys_cap + 2)) - 1);
            (void)locali_cache_probation_size(c);
            (void)locali_cache_protected_size(c);
        }
        locali_cache_destroy(c);
    }
    puts("fuzz ok");
    return 0;
}
