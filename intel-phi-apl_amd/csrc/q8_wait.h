/* q8_wait.h: the runtime's one way of waiting for the GPU, with a deadline.
 *
 * Every host wait of the library (a product's completion flag, a stream or an event) polls until
 * the work is done or `deadline_s` seconds have passed. Past the deadline it prints what it was
 * waiting for and how long it waited, and ends the process with _exit(3): a kernel that never
 * ends stops the engine with a message instead of hanging it. The reference never blocks forever
 * either: its card exits with status 3 after about 60 s without the host
 * (src/card/link.c:17-32) and its stream gives up after 120 s (src/card/stream.c:63-70).
 *
 * Host code only (no HIP types), so that a CPU test can drive the loop with a poll that never
 * completes (tests/c/wait_deadline.cpp). */
#ifndef Q8_WAIT_H
#define Q8_WAIT_H

#include <stdio.h>
#include <unistd.h>

#include <chrono>

/* The deadline when Q8_WAIT_S is not set (seconds). */
#define Q8_WAIT_DEFAULT_S 60.0

/* Polls poll() (true once the work is done; it may itself stop the process on an error) until it
 * returns true. For the first 2 ms between polls the thread only pauses, so that a product's
 * completion is seen within a few hundred nanoseconds; after that it sleeps 20 us between polls.
 * Past deadline_s seconds: the message on stderr, then _exit(3). */
template <class Poll>
inline void q8_wait_until(Poll &&poll, double deadline_s, const char *what)
{
    using clock = std::chrono::steady_clock;
    const clock::time_point t0 = clock::now();
    for (unsigned long spins = 0;; spins++) {
        if (poll())
            return;
        if ((spins & 63) != 63) {
            __builtin_ia32_pause();
            continue;
        }
        const double waited = std::chrono::duration<double>(clock::now() - t0).count();
        if (waited > deadline_s) {
            fprintf(stderr, "q8_rt: %s did not complete within %.1f s (the deadline, Q8_WAIT_S): the GPU work it waits for never ended; exiting with status 3\n",
                    what, waited);
            fflush(stderr);
            _exit(3);
        }
        if (waited > 0.002)
            usleep(20);
    }
}

#endif
