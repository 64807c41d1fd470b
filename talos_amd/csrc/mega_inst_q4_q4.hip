// mega_inst_q4_q4.hip -- k_mega instantiations (see mega_inst.h).
#include "mega.h"
#include "mega_inst.h"

const void* mega_inst_q4_q4(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm) {
  MEGA_PICK(TALOS_FMT_Q4_0, TALOS_FMT_Q4_0, 2, 4, 2, 8, MEGA_MM_DOT4);
  MEGA_PICK(TALOS_FMT_Q4_0, TALOS_FMT_Q4_0, 2, 2, 2, 8, MEGA_MM_F32);
  return nullptr;
}
