/* Drives the library's wait loop (intel-phi-apl_amd/csrc/q8_wait.h) on the CPU with polls of known
 * behaviour: argv[1] = "done" (completes on the 1000th poll), "slow" (completes after 50 ms, past
 * the loop's busy phase), "never" (never completes: the loop must end the process with status 3
 * and its message once argv[2] seconds have passed). */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>

#include "q8_wait.h"

int main(int argc, char **argv)
{
    if (argc < 3)
        return 2;
    const double deadline = atof(argv[2]);
    const auto t0 = std::chrono::steady_clock::now();
    auto since = [&] { return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count(); };
    long polls = 0;
    if (strcmp(argv[1], "done") == 0)
        q8_wait_until([&] { return ++polls >= 1000; }, deadline, "the done case");
    else if (strcmp(argv[1], "slow") == 0)
        q8_wait_until([&] { ++polls; return since() > 0.05; }, deadline, "the slow case");
    else if (strcmp(argv[1], "never") == 0)
        q8_wait_until([&] { ++polls; return false; }, deadline, "the never case");
    else
        return 2;
    printf("returned after %ld polls, %.3f s\n", polls, since());
    return 0;
}
