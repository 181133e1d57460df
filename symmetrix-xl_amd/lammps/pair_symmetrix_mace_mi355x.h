/* -*- c++ -*- ----------------------------------------------------------
   pair_style symmetrix/mace/mi355x/kk: MACE energies, forces and virial on
   one MI355X through libsymmetrix_mi355x.so (include/symmetrix_mi355x.h).

   Two of the reference's pair_style symmetrix/mace/kk modes:
   * no_domain_decomposition (one MPI rank; pair_symmetrix_mace_kokkos.cpp:
     1010-1282): one full Kokkos neighbour list with ghosts, every local atom
     a graph node, every neighbour (local or ghost) an edge to the local atom
     it is an image of.  The library builds the graph on neighbour-list
     rebuilds, forms the edge vectors from x each step, evaluates the model
     and adds the edge forces to the local and ghost rows of f (the ghost rows
     then go through LAMMPS's reverse communication).
   * mpi_message_passing (one rank per GPU; :1285-1704): each rank's local
     atoms are the receivers and every local or ghost atom a feature node of
     the library's split-phase evaluation; between its phases the H1 rows of
     the ghosts come from their owners (forward communication) and the H1
     adjoint rows of the ghosts go back to them (reverse communication).
   The default is no_domain_decomposition on one rank and
   mpi_message_passing on several.

   Usage (the reference's keywords where they apply):
     pair_style symmetrix/mace/mi355x/kk [no_domain_decomposition|mpi_message_passing] [head NAME]
                [profile capacity|speed] [low_memory yes|no]
                [allow_fixed_workspace yes|no] [streamed_edges auto|direct]
                [electric_field Ex Ey Ez]   (required by MACEField models)
     pair_coeff * * model.json O Ti Sr      (one element symbol per LAMMPS type)
   Requires newton pair on and an atom map.

   Built as a LAMMPS KOKKOS package style for HIP (Kokkos_ENABLE_HIP) linked
   against libsymmetrix_mi355x.so.  This repository has no LAMMPS sources:
   its tests type-check the class against stand-ins of the LAMMPS and Kokkos
   declarations it uses (tests/lammps_stub).
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

  // H1 rows forward, H1 adjoint rows in reverse (mpi_message_passing)
  int pack_forward_comm_kokkos(int, DAT::tdual_int_1d, DAT::tdual_double_1d &, int, int *) override;
  void unpack_forward_comm_kokkos(int, int, DAT::tdual_double_1d &) override;
  int pack_reverse_comm_kokkos(int, int, DAT::tdual_double_1d &) override;
  void unpack_reverse_comm_kokkos(int, DAT::tdual_int_1d, DAT::tdual_double_1d &) override;
  int pack_forward_comm(int, int *, double *, int, int *) override;
  void unpack_forward_comm(int, int, double *) override;
  int pack_reverse_comm(int, int, double *) override;
  void unpack_reverse_comm(int, int *, double *) override;

 protected:
  SmxEvaluator *evaluator = nullptr;
  std::string head;
  std::string debug_plan;
  std::string execution_profile = "capacity";
  bool allow_fixed_workspace = false;
  double electric_field[3] = {0.0, 0.0, 0.0};  // electric_field Ex Ey Ez (MACEField models)
  bool electric_field_set = false;
  double r_cut = 0.0;

  std::string mode;                 // no_domain_decomposition or mpi_message_passing
  bool single_layer = false;        // one-interaction model: no features are exchanged
  int row_floats = 0;               // FP32 values of one atom's H1 row
  uint64_t generation = 0;          // the rank's feature graph (mpi_message_passing)
  int graph_nall = -1;
  int64_t num_edges = 0;
  Kokkos::View<int *, DeviceType> d_feature_types, d_receiver_features, d_node_types, d_num_neigh, d_first,
      d_neigh, d_neigh_types;
  Kokkos::View<float *, DeviceType> d_h1;          // [nall][row_floats] H1 rows by LAMMPS index
  float *exchange_rows = nullptr;                   // the evaluator's H1 adjoint rows while they are exchanged
  Kokkos::View<double *, DeviceType> d_stage;       // host-staged communication
  Kokkos::View<int *, DeviceType> d_stage_list;

  Kokkos::View<int *, DeviceType> d_type_to_model;  // [ntypes] model type of LAMMPS type t+1
  Kokkos::View<int *, DeviceType> d_owner;          // [nall] local atom each atom is an image of
  typename Kokkos::View<int *, DeviceType>::HostMirror h_owner;
  DAT::tdual_efloat_1d k_eatom;

  void allocate();
  void check(int32_t status, const char *what);
  void compute_no_domain_decomposition();
  void compute_mpi_message_passing();
  void stage(size_t values);
};

}    // namespace LAMMPS_NS

#endif
#endif
