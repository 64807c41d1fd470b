// mega_inst_q8_wide.hip -- k_mega instantiations (see mega_inst.h).
#include "mega.h"
#include "mega_inst.h"

const void* mega_inst_q8_wide(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm) {
  MEGA_PICK(TALOS_FMT_Q8_0, TALOS_FMT_Q8_0, 2, 2, 2, 8, MEGA_MM_DOT4);
  MEGA_PICK(TALOS_FMT_Q8_0, TALOS_FMT_Q8_0, 2, 2, 2, 8, MEGA_MM_F32);
  return nullptr;
}
