// mega_inst.h -- the persistent-kernel instantiations this library carries.
//
// Each mega_inst_*.hip translation unit instantiates a few k_mega
// specialisations (mega.h) and returns the one matching a request, so the
// heavy kernels compile in parallel.  A request names the layer and output
// formats, the chunk-steps per item of the n-, ff- and output-wide rows,
// head_dim / 16 and the matvec mode (MEGA_MM_*).
#pragma once
#include <stdint.h>

typedef const void* (*MegaInstFn)(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm);

const void* mega_inst_q4_mfma(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm);
const void* mega_inst_q4_q6k(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm);
const void* mega_inst_q4_q4(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm);
const void* mega_inst_q8_wide(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm);
const void* mega_inst_q8_small(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm);
const void* mega_inst_f32(uint32_t lf, uint32_t of, int un, int uf, int uo, int dpl, int mm);

#define MEGA_INST_FNS \
  {mega_inst_q4_mfma, mega_inst_q4_q6k, mega_inst_q4_q4, mega_inst_q8_wide, mega_inst_q8_small, mega_inst_f32}

// The kernel address of k_mega<LF, OF, UN, UF, UO, DPL, MM> when the request
// is exactly that tuple, else null (used inside the instantiating units).
#define MEGA_PICK(LF, OF, UN, UF, UO, DPL, MM)                                                   \
  if (lf == (LF) && of == (OF) && un == (UN) && uf == (UF) && uo == (UO) && dpl == (DPL) &&      \
      mm == (MM))                                                                                 \
    return (const void*)k_mega<LF, OF, UN, UF, UO, DPL, MM>;
