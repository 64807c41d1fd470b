// mega_inst_f32.hip -- k_mega instantiations (see mega_inst.h).
#include "mega.h"
#include "mega_inst.h"

const void* mega_inst_f32(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm) {
  MEGA_PICK(TALOS_FMT_F32, TALOS_FMT_F32, 2, 2, 2, 3, MEGA_MM_F32);
  return nullptr;
}
