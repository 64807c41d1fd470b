// mega_inst_q8_small.hip -- k_mega instantiations (see mega_inst.h).
#include "mega.h"
#include "mega_inst.h"

const void* mega_inst_q8_small(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm) {
  MEGA_PICK(TALOS_FMT_Q8_0, TALOS_FMT_Q8_0, 1, 1, 1, 4, MEGA_MM_DOT4);
  MEGA_PICK(TALOS_FMT_Q8_0, TALOS_FMT_Q8_0, 1, 1, 1, 4, MEGA_MM_F32);
  return nullptr;
}
