// ref_contracts.cpp — runs the reference's own header-only contract helpers
// over a sweep of inputs and prints their answers as JSON lines, so the
// tests can hold the Python oracle (oracle/kv_oracle.py) against them.
//
// TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile from the reference
// headers where they lie (never copied):
//   native/gemma4_listener_microbatch/gemma4_listener_batch_contract.h:228-282
//     gemma4_history_batch_make_plan / _causal_key_limit / _sliding_start
//   native/gemma4_listener_microbatch/sliding_repeat_capacity.h:30-60
//     gemma4_sliding_staging::derive_contract
// Output goes to oracle/_ref/ (git-ignored).
#include <cstdio>
#include <cstring>

#include "gemma4_listener_batch_contract.h"
#include "sliding_repeat_capacity.h"

int main() {
    // Causal key limit and sliding start of every query of a history batch.
    const uint32_t prefixes[] = {1, 4, 91, 265, 511, 512, 777, 1000};
    const uint32_t audio[] = {4, 8, 36, 256};
    const uint32_t windows[] = {1, 2, 128, 512};
    for (uint32_t prefix : prefixes) {
        for (uint32_t a : audio) {
            gemma4_history_batch_plan plan{};
            if (!gemma4_history_batch_make_plan(prefix, prefix, prefix, a, 4096, prefix > a ? prefix : a, 256,
                                                4096, &plan))
                continue;
            for (uint32_t qi = 0; qi < a; ++qi) {
                std::printf("{\"kind\": \"causal\", \"prefix\": %u, \"q\": %u, \"limit\": %u}\n", prefix, qi,
                            gemma4_history_batch_causal_key_limit(&plan, qi));
                for (uint32_t w : windows)
                    std::printf("{\"kind\": \"sliding\", \"prefix\": %u, \"q\": %u, \"window\": %u, \"start\": %u}\n",
                                prefix, qi, w, gemma4_history_batch_sliding_start(&plan, qi, w));
            }
        }
    }
    // Rows a sliding layer must keep for (window, max query, max_seq_len).
    const uint32_t cap_windows[] = {1, 64, 512, 1024};
    const uint32_t max_q[] = {1, 2, 8, 291};
    const uint32_t max_seq[] = {16, 600, 802, 16384};
    for (uint32_t w : cap_windows)
        for (uint32_t q : max_q)
            for (uint32_t s : max_seq) {
                GemmaLayerSpec layers[2];
                std::memset(layers, 0, sizeof(layers));
                layers[0].attn_type = GEMMA_ATTN_SLIDING;
                layers[0].head_dim = 256;
                layers[0].sliding_window = w;
                layers[1].attn_type = GEMMA_ATTN_FULL;
                layers[1].head_dim = 512;
                gemma4_sliding_staging::Contract c{};
                const bool ok = gemma4_sliding_staging::derive_contract(layers, 2, s, q, &c);
                std::printf("{\"kind\": \"capacity\", \"window\": %u, \"max_q\": %u, \"max_seq\": %u, \"ok\": %s, "
                            "\"capacity\": %u}\n", w, q, s, ok ? "true" : "false", c.capacity);
            }
    return 0;
}
