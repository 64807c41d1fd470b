// mega_inst_q4_mfma.hip -- k_mega instantiations (see mega_inst.h).
#include "mega.h"
#include "mega_inst.h"

const void* mega_inst_q4_mfma(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm) {
  MEGA_PICK(TALOS_FMT_Q4_0, TALOS_FMT_Q6_K, 4, 14, 1, 8, MEGA_MM_MFMA);
  return nullptr;
}
