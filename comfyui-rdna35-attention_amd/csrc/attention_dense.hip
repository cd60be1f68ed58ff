// The dense attention launchers and kernels (exact attention over every key
// block, no tail): attention.hip compiled with PISA_ATTENTION_DENSE, built with
// the max-memory-clause machine scheduler (build_lib.py).
#define PISA_ATTENTION_DENSE 1
#include "attention.hip"
