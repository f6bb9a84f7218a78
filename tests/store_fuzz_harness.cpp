// Host-only harness for tests/test_store_fuzz.py: opens every store named on
// the command line with qf_store_open (built from qfm_store.cpp with the
// address and undefined-behaviour sanitizers), reads the first and last byte
// of every entry of the stores that open, closes them, and prints the counts.
#include "../include/qf_store.h"
#include <cstdarg>
#include <cstdio>

namespace qfm {
// the library's error latch and configuration, reduced to what the reader uses
struct Cfg { int H = 2048, I = 512, E = 512, K = 10, renorm = 1, gated = 1; };
Cfg g_cfg;
static char g_msg[512];
void set_error(int, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof g_msg, fmt, ap);
    va_end(ap);
}
int check_launch(const char *) { return 0; }
}  // namespace qfm

int main(int argc, char **argv) {
    int opened = 0, rejected = 0;
    for (int i = 1; i < argc; i++) {
        QfStore st{};
        if (qf_store_open(&st, argv[i]) != 0) {
            rejected++;
            continue;
        }
        opened++;
        for (int e = 0; e < st.n_entries; e++) {
            const QfEntry *en = qf_find(&st, st.entries[e].name);
            if (!en) {
                printf("lookup of %s failed\n", st.entries[e].name);
                return 2;
            }
            const unsigned char *p = static_cast<const unsigned char *>(qfm_store_data(&st, en));
            volatile unsigned sink = 0;
            if (p && en->rec.nbytes) sink += p[0] + p[en->rec.nbytes - 1];
        }
        qf_store_close(&st);
    }
    printf("opened %d rejected %d\n", opened, rejected);
    return 0;
}
