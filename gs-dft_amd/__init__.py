"""MI355X-native screened density-fitted Coulomb (DF-J) for floating anisotropic Gaussian splats.

A drop-in for the DF-J path of gs-dft and its neighbours on the same pair list (screened RI-K,
exact screened Coulomb, nuclear attraction, density on the XC grid): the ``df()`` /
``pairlist()`` plugin surface, the ``SplatState`` refresh contract and
``ScreenedProductDFCoulomb.energy``, backed by hand-written HIP kernels for gfx950 in ``lib/libgsdft.so`` (C ABI declared in ``include/gsdft.h``).
"""
from .basis import IsotropicSplat, Splat, init_product_aux
from .energy import SplatDFJ, SplatModel, SplatState, refresh, train_pad_to
from .exact import (full_coulomb_J, full_coulomb_energy, make_pairs, screened_coulomb_J,
                    screened_coulomb_energy)
from .grid import chunked_density, chunked_density_and_grad, chunked_density_grad_tau
from .ri import (aux_cholesky, aux_metric, coulomb_pairs, df_coulomb_energy_screened,
                 df_coulomb_gamma_screened, df_coulomb_solve, df_exchange_energy_screened,
                 shift_diag)
from .screening import (PairIndex, build_pair_index, count_significant, density_pairs,
                        live_length, neighbor_pairs, pair_weight, screened_external_energy,
                        screened_nuclear_pairs, screened_overlap_pairs)
from .terms import (SCREEN_PAD, CoulombTerm, DFSpec, ExactSpec, Pairlist, ScreenedExactCoulomb,
                    ScreenedProductDFCoulomb, StreamedExactCoulomb, df, exact, hf_coeff, pairlist)

__all__ = [
    "Splat", "IsotropicSplat", "init_product_aux",
    "SplatDFJ", "SplatModel", "SplatState", "refresh", "train_pad_to",
    "aux_metric", "aux_cholesky", "shift_diag", "df_coulomb_gamma_screened", "df_coulomb_solve",
    "df_coulomb_energy_screened", "coulomb_pairs", "df_exchange_energy_screened",
    "screened_coulomb_energy", "screened_coulomb_J", "full_coulomb_energy", "full_coulomb_J",
    "make_pairs",
    "chunked_density", "chunked_density_and_grad", "chunked_density_grad_tau",
    "neighbor_pairs", "count_significant", "pair_weight", "screened_overlap_pairs",
    "density_pairs", "screened_nuclear_pairs", "screened_external_energy",
    "PairIndex", "build_pair_index", "live_length",
    "SCREEN_PAD", "CoulombTerm", "DFSpec", "ExactSpec", "Pairlist", "ScreenedProductDFCoulomb",
    "ScreenedExactCoulomb", "StreamedExactCoulomb",
    "df", "exact", "pairlist", "hf_coeff",
]
