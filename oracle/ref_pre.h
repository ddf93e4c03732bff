/* ref_pre.h -- prepended when oracle/Makefile compiles the GEMM path of
 * /root/reference/tinylm.c straight from that file (lines streamed into gcc's
 * stdin; no reference text is stored in this repository).
 *
 * TEST INFRASTRUCTURE ONLY.  These are the standard headers tinylm.c:19-32
 * includes, minus <direct.h>: that header (and the Win32 imports) serve the
 * CLI and file I/O, which the compiled line ranges do not contain.  Nothing
 * here stands in for a missing header or library. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <stdint.h>
#include <time.h>
#include <omp.h>
#include <immintrin.h>
