/* -*- c++ -*- ----------------------------------------------------------
   pair_style symmetrix/mace/mi355x/kk: MACE energies, forces and virial on
   one MI355X through libsymmetrix_mi355x.so (include/symmetrix_mi355x.h).

   The single-rank path of the reference's pair_style symmetrix/mace/kk
   without domain decomposition (pair_symmetrix_mace_kokkos.cpp:1010-1282):
   one full Kokkos neighbour list with ghosts, every local atom a graph
   node, every neighbour (local or ghost) an edge to the local atom it is an
   image of.  The library builds the graph on neighbour-list rebuilds, forms
   the edge vectors from x each step, evaluates the model and adds the edge
   forces to the local and ghost rows of f (the ghost rows then go through
   LAMMPS's reverse communication).

   Usage (the reference's keywords where they apply):
     pair_style symmetrix/mace/mi355x/kk [no_domain_decomposition] [head NAME]
                [profile capacity|speed] [low_memory yes|no]
                [allow_fixed_workspace yes|no] [streamed_edges auto|direct]
                [electric_field Ex Ey Ez]   (required by MACEField models)
     pair_coeff * * model.json O Ti Sr      (one element symbol per LAMMPS type)
   Requires newton pair on and an atom map.

   Built as a LAMMPS KOKKOS package style for HIP (Kokkos_ENABLE_HIP) linked
   against libsymmetrix_mi355x.so; not compiled in this repository, which
   has no LAMMPS sources.
------------------------------------------------------------------------- */

#ifdef PAIR_CLASS
// clang-format off
PairStyle(symmetrix/mace/mi355x/kk,PairSymmetrixMACEMI355X<LMPDeviceType>);
// clang-format on
#else

#ifndef LMP_PAIR_SYMMETRIX_MACE_MI355X_H
#define LMP_PAIR_SYMMETRIX_MACE_MI355X_H

#include <string>
#include <vector>

#include "kokkos_base.h"
#include "neigh_list_kokkos.h"
#include "pair_kokkos.h"
#include "symmetrix_mi355x.h"

namespace LAMMPS_NS {

template <class DeviceType>
class PairSymmetrixMACEMI355X : public Pair, public KokkosBase {
 public:
  typedef DeviceType device_type;
  typedef ArrayTypes<DeviceType> AT;

  explicit PairSymmetrixMACEMI355X(class LAMMPS *);
  ~PairSymmetrixMACEMI355X() override;

  void compute(int, int) override;
  void settings(int, char **) override;
  void coeff(int, char **) override;
  double init_one(int, int) override;
  void init_style() override;

 protected:
  SmxEvaluator *evaluator = nullptr;
  std::string head;
  std::string debug_plan;
  std::string execution_profile = "capacity";
  bool allow_fixed_workspace = false;
  double electric_field[3] = {0.0, 0.0, 0.0};  // electric_field Ex Ey Ez (MACEField models)
  bool electric_field_set = false;
  double r_cut = 0.0;

  Kokkos::View<int *, DeviceType> d_type_to_model;  // [ntypes] model type of LAMMPS type t+1
  Kokkos::View<int *, DeviceType> d_owner;          // [nall] local atom each atom is an image of
  typename Kokkos::View<int *, DeviceType>::HostMirror h_owner;
  DAT::tdual_efloat_1d k_eatom;

  void allocate();
  void check(int32_t status, const char *what);
};

}    // namespace LAMMPS_NS

#endif
#endif
