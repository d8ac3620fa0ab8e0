// Bits of the int4 `flags` argument that are not part of the public ABI.
//
// The public value is 0 (include/xk_moe.h). The bits below pick a kernel where
// the shapes allow more than one, so the GPU tests can compare the prefill tile
// kernel with the decode stream kernel on the same inputs. Callers outside the
// tests leave them clear; any other bit is rejected.
#pragma once

#define XK_INT4_TEST_FORCE_TILE (1 << 8)
#define XK_INT4_TEST_FORCE_STREAM (1 << 9)
