// SPDX-License-Identifier: MIT
// The expert-stack ledger across several live backends, called directly (it has no ABI entry):
// the cases of test-rocket-internals.cpp:155-215 restated for an HBM copy per backend (the NPU's
// IOVA window and its separate GGUF-source charge do not exist here: a copy's charge is its HBM
// bytes). Built and run by tests/test_internals.py with the host sources it exercises.
#include <stdio.h>
#include <stdlib.h>

#include "../../ggml-rocket_amd/csrc/host/host.h"

using namespace mxh;

static int g_fails = 0;
#define CHECK(cond, what)                                      \
    do {                                                       \
        if (cond) printf("ok   %s\n", what);                   \
        else { printf("FAIL %s\n", what); g_fails++; }         \
    } while (0)

int main() {
    // 80 MB budget: one 40 MB stack copy fits, a second copy of it too, a third does not
    setenv("MI355X_MOE_CACHE_MB", "80", 1);
    const size_t big = (size_t)40 << 20, small = (size_t)9 << 20;

    moe_preflight_open();   // backend A
    moe_preflight_open();   // backend B
    CHECK(moe_preflight_admit("big", big, nullptr, 0), "placement admits the big stack (one spare copy charged)");
    bool placed = false;
    CHECK(moe_preflight_decided("big", &placed) && placed, "the decision is remembered");
    CHECK(moe_preflight_claim("big") == MOE_CLAIMED, "backend A takes the spare copy");
    CHECK(moe_preflight_claim("big") == MOE_CLAIMED, "backend B's own copy fits (80 MB charged)");
    CHECK(!moe_preflight_admit("small", small, nullptr, 0), "a new stack past the budget is declined whole");
    CHECK(moe_preflight_decided("small", &placed) && !placed, "and the decline is remembered");
    CHECK(moe_preflight_claim("small") == MOE_UNDECIDED, "a declined stack has no copy to take");
    moe_preflight_open();   // backend C
    CHECK(moe_preflight_claim("big") == MOE_REFUSED, "backend C's copy would pass the budget: refused");
    moe_preflight_release("big");   // backend A freed
    moe_preflight_close();
    CHECK(moe_preflight_claim("big") == MOE_CLAIMED, "A's returned copy makes room for C");
    CHECK(moe_preflight_decided("big", &placed) && placed, "claims and returns leave the decision alone");
    CHECK(!moe_preflight_admit("small", small, nullptr, 0), "the remembered decline stands while backends live");
    moe_preflight_release("big");
    moe_preflight_close();   // B
    moe_preflight_release("big");
    moe_preflight_close();   // C
    moe_preflight_open();    // a fresh backend: the ledger starts over
    CHECK(!moe_preflight_decided("big", &placed), "the ledger is forgotten once no backend is live");
    CHECK(moe_preflight_admit("small", small, nullptr, 0), "and a stack declined before is decided again");
    CHECK(moe_preflight_claim("small") == MOE_CLAIMED, "its spare copy is taken");
    CHECK(moe_preflight_claim("nobody") == MOE_UNDECIDED && !moe_preflight_admit("", big, nullptr, 0),
          "an unknown or unnamed stack is neither placed nor claimed");
    moe_preflight_release("small");
    moe_preflight_close();
    printf("%d failed\n", g_fails);
    return g_fails ? 1 : 0;
}
