// Drives gsv_ar::generate (include/gsv_ar.h, linked from libgsvk.so) on an AR GGUF and prints the
// engine's progress counters (include/gsv_progress.h) as this program sees them afterwards: one
// object per process, so the library's ticks show here as they would in the engine's server.
#include <cstdio>
#include <vector>

#include "gsv_ar.h"
#include "gsv_progress.h"

int main(int argc, char ** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s ar.gguf\n", argv[0]);
        return 2;
    }
    gsv_ar * ar = gsv_ar::load(argv[1], gsv_ar_cfg());
    if (!ar) return 3;
    gsv_ar_request r;
    for (int i = 0; i < 12; i++) r.phones.push_back(5 + 7 * i);
    for (int i = 0; i < 8; i++) r.prompt.push_back(100 + 3 * i);
    const int max_steps = 17;
    gsvprog::begin(0, 0);
    const gsv_ar_result res = ar->generate({r}, gsv_sampler_cfg(), 1234, -1, max_steps);
    if (res.tokens.size() != 1) return 4;
    const int generated = (int) res.tokens[0].size() - (int) r.prompt.size();
    printf("progress %d %d %d %d\n", gsvprog::stage.load(), gsvprog::cur.load(), gsvprog::total.load(), generated);
    delete ar;
    return 0;
}
