# The edit that lets fpedd/l3m's dispatcher (src/dispatch.c) pick the "hip" kernel table of libl3m_hip.so,
# applied to the reference's file as it streams into the compiler (oracle/Makefile, _ref/libl3m_ref_hip.so).
# Each command appends one line after a line of dispatch.c, found by its text:
#  - after the include of kernels.h: the table and the library's usability check (a maintainer would put
#    the table into kernels.h's extern list, kernels.h:42, instead);
#  - first in l3m_kernels_usable (dispatch.c:23): the library answers for its own table;
#  - in l3m_kernels_pick, once L3M_ISA is read (dispatch.c:30): L3M_ISA=hip takes the table when a GPU is
#    usable; otherwise the dispatcher goes on as before, to its message and its best CPU table.
/^#include "kernels.h"$/a\
extern const l3m_kernels l3m_kernels_hip;\
int l3m_hip_kernels_usable(void);
/^int l3m_kernels_usable(const l3m_kernels \*k) {/a\
    if (k == &l3m_kernels_hip) return l3m_hip_kernels_usable();
/^    const char \*want = getenv("L3M_ISA");$/a\
    if (want && !strcmp(want, "hip") && l3m_hip_kernels_usable()) return &l3m_kernels_hip;
