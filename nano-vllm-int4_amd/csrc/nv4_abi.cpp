// Library-level entry points of libnv4.so (version and error text).
#include "../../include/nv4.h"

extern "C" const char* nv4_version(void) { return "nv4 0.1.0 gfx950"; }

extern "C" const char* nv4_strerror(int code) {
    switch (code) {
        case NV4_OK: return "ok";
        case NV4_E_NULL: return "a required pointer is NULL";
        case NV4_E_SHAPE: return "unsupported shape";
        case NV4_E_ALIGN: return "misaligned pointer";
        case NV4_E_LAYOUT: return "unknown rotation layout";
        case NV4_E_DTYPE: return "unknown dtype code";
        case NV4_E_GROUP: return "unsupported group size";
        case NV4_E_SCRATCH: return "needs more device scratch than the allocation-free entry point has";
        default: return code > 0 ? "hip error" : "unknown error";
    }
}
