/* ----------------------------------------------------------------------
   pair_style symmetrix/mace/mi355x/kk (see pair_symmetrix_mace_mi355x.h)

   no_domain_decomposition follows the reference's path of that name
   (pair_symmetrix_mace_kokkos.cpp:1010-1282) with the work inside
   smx_lammps_compute: graph on rebuilds, edge vectors from x, model,
   deterministic force gather onto local and ghost rows, per-atom energies and
   the virial.  The call is ordered after the work Kokkos queued on the
   execution space's stream (SmxLammpsArgsV2.stream).

   mpi_message_passing follows :1285-1704: a feature graph of the rank's
   local atoms (receivers) and all its local and ghost atoms (feature nodes,
   by LAMMPS index) on rebuilds, edge vectors each step, then the library's
   split phases with LAMMPS's forward communication of H1 rows between begin
   and continue and the reverse communication of H1 adjoint rows between
   continue and finish; feature-node forces go to the local and ghost rows
   of f.  Communicated values are doubles, as LAMMPS buffers are.
------------------------------------------------------------------------- */

#include "pair_symmetrix_mace_mi355x.h"

#include "atom_kokkos.h"
#include "atom_masks.h"
#include "comm.h"
#include "error.h"
#include "force.h"
#include "kokkos.h"
#include "memory_kokkos.h"
#include "neigh_request.h"
#include "neighbor.h"
#include "utils.h"

#include <climits>
#include <cstdlib>
#include <cstring>

using namespace LAMMPS_NS;

namespace {
// atomic number of an element symbol (0: not an element)
int element_number(const char *symbol)
{
  static const char *const kSymbols[] = {
      "H",  "He", "Li", "Be", "B",  "C",  "N",  "O",  "F",  "Ne", "Na", "Mg", "Al", "Si", "P",
      "S",  "Cl", "Ar", "K",  "Ca", "Sc", "Ti", "V",  "Cr", "Mn", "Fe", "Co", "Ni", "Cu", "Zn",
      "Ga", "Ge", "As", "Se", "Br", "Kr", "Rb", "Sr", "Y",  "Zr", "Nb", "Mo", "Tc", "Ru", "Rh",
      "Pd", "Ag", "Cd", "In", "Sn", "Sb", "Te", "I",  "Xe", "Cs", "Ba", "La", "Ce", "Pr", "Nd",
      "Pm", "Sm", "Eu", "Gd", "Tb", "Dy", "Ho", "Er", "Tm", "Yb", "Lu", "Hf", "Ta", "W",  "Re",
      "Os", "Ir", "Pt", "Au", "Hg", "Tl", "Pb", "Bi", "Po", "At", "Rn", "Fr", "Ra", "Ac", "Th",
      "Pa", "U",  "Np", "Pu", "Am", "Cm", "Bk", "Cf", "Es", "Fm", "Md", "No", "Lr", "Rf", "Db",
      "Sg", "Bh", "Hs", "Mt", "Ds", "Rg", "Cn", "Nh", "Fl", "Mc", "Lv", "Ts", "Og"};
  for (int z = 0; z < 118; ++z)
    if (strcmp(symbol, kSymbols[z]) == 0) return z + 1;
  return 0;
}
}    // namespace

template <class DeviceType>
PairSymmetrixMACEMI355X<DeviceType>::PairSymmetrixMACEMI355X(LAMMPS *lmp) : Pair(lmp)
{
  respa_enable = 0;
  kokkosable = 1;
  atomKK = (AtomKokkos *) atom;
  execution_space = ExecutionSpaceFromDevice<DeviceType>::space;
  datamask_read = X_MASK | F_MASK | TYPE_MASK | TAG_MASK | ENERGY_MASK | VIRIAL_MASK;
  datamask_modify = F_MASK | ENERGY_MASK | VIRIAL_MASK;
  no_virial_fdotr_compute = 1;
  one_coeff = 1;
  manybody_flag = 1;
  reverse_comm_device = 1;
}

template <class DeviceType>
PairSymmetrixMACEMI355X<DeviceType>::~PairSymmetrixMACEMI355X()
{
  if (copymode) return;
  if (evaluator) smx_evaluator_destroy(evaluator);
  memoryKK->destroy_kokkos(k_eatom, eatom);
  if (allocated) {
    memory->destroy(setflag);
    memory->destroy(cutsq);
  }
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::check(int32_t status, const char *what)
{
  if (status != SMX_OK) error->all(FLERR, "symmetrix/mace/mi355x {}: {}", what, smx_last_error());
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::allocate()
{
  allocated = 1;
  const int n = atom->ntypes;
  memory->create(setflag, n + 1, n + 1, "pair:setflag");
  memory->create(cutsq, n + 1, n + 1, "pair:cutsq");
  for (int i = 1; i <= n; i++)
    for (int j = i; j <= n; j++) setflag[i][j] = 0;
}

// The reference's keywords (pair_symmetrix_mace_kokkos.cpp:180-370) where
// this build has them: the mode token (no_domain_decomposition or
// mpi_message_passing), profile capacity|speed and its low_memory yes|no alias, allow_fixed_workspace
// yes|no, head NAME, streamed_edges auto|direct, _debug_execution_plan ID,
// electric_field Ex Ey Ez (MACEField, :207-224).  The JIT artefact keywords
// name files this build does not load (warned and skipped);
// no_mpi_message_passing (ghost neighbour lists) is refused.
template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::settings(int narg, char **arg)
{
  mode = comm->nprocs == 1 ? "no_domain_decomposition" : "mpi_message_passing";
  execution_profile = "capacity";
  allow_fixed_workspace = false;
  head.clear();
  debug_plan.clear();
  electric_field_set = false;
  bool profile_set = false, alias_set = false;
  std::string alias_profile;
  auto value_of = [&](int &i, const char *what) -> std::string {
    if (i + 1 >= narg) error->all(FLERR, "pair_style symmetrix/mace/mi355x/kk {} requires a value", what);
    return arg[++i];
  };
  auto yes_no = [&](const std::string &key, const std::string &v) {
    if (v != "yes" && v != "no")
      error->all(FLERR, "pair_style symmetrix/mace/mi355x/kk {} requires yes or no", key);
    return v == "yes";
  };
  for (int i = 0; i < narg; ++i) {
    const std::string key = arg[i];
    if (key == "no_domain_decomposition" || key == "mpi_message_passing") {
      mode = key;
    } else if (key == "no_mpi_message_passing") {
      error->all(FLERR, "pair_style symmetrix/mace/mi355x/kk has no {} mode", key);
    } else if (key == "profile") {
      execution_profile = value_of(i, "profile");
      if (execution_profile != "capacity" && execution_profile != "speed")
        error->all(FLERR, "pair_style symmetrix/mace/mi355x/kk profile requires capacity or speed");
      profile_set = true;
    } else if (key == "low_memory") {
      alias_profile = yes_no(key, value_of(i, "low_memory")) ? "capacity" : "speed";
      alias_set = true;
    } else if (key == "allow_fixed_workspace") {
      allow_fixed_workspace = yes_no(key, value_of(i, "allow_fixed_workspace"));
    } else if (key == "head") {
      head = value_of(i, "head");
    } else if (key == "streamed_edges") {
      const std::string v = value_of(i, "streamed_edges");
      if (v != "auto" && v != "direct")
        error->all(FLERR, "pair_style symmetrix/mace/mi355x/kk streamed_edges runs auto or direct only");
    } else if (key == "_debug_execution_plan") {
      debug_plan = value_of(i, "_debug_execution_plan");
    } else if (key.rfind("jit_", 0) == 0) {
      const std::string v = value_of(i, key.c_str());
      if (comm->me == 0) error->warning(FLERR, "pair_style symmetrix/mace/mi355x/kk ignores {} {}", key, v);
    } else if (key == "electric_field") {
      if (i + 3 >= narg) error->all(FLERR, "pair_style symmetrix/mace/mi355x/kk electric_field requires three components");
      for (int c = 0; c < 3; ++c) {
        char *end = nullptr;
        electric_field[c] = std::strtod(arg[i + 1 + c], &end);
        if (end == arg[i + 1 + c] || *end != '\0')
          error->all(FLERR, "pair_style symmetrix/mace/mi355x/kk electric_field components must be numeric");
      }
      i += 3;
      electric_field_set = true;
    } else {
      error->all(FLERR, "The command 'pair_style symmetrix/mace/mi355x/kk {}' is invalid", key);
    }
  }
  if (alias_set) {
    if (profile_set && execution_profile != alias_profile)
      error->all(FLERR, "pair_style symmetrix/mace/mi355x/kk low_memory contradicts profile");
    execution_profile = alias_profile;
  }
  if (mode == "no_domain_decomposition" && comm->nprocs != 1)
    error->all(FLERR, "Cannot use no_domain_decomposition with multiple MPI processes");
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::coeff(int narg, char **arg)
{
  if (!allocated) allocate();
  if (narg != atom->ntypes + 3) error->all(FLERR, "Incorrect args for pair coefficients");
  if (strcmp(arg[0], "*") != 0 || strcmp(arg[1], "*") != 0)
    error->all(FLERR, "pair_coeff for symmetrix/mace/mi355x/kk must be '* * model.json elements...'");
  if (evaluator) smx_evaluator_destroy(evaluator);
  utils::logmesg(lmp, "Loading MACE model from '{}' on the MI355X evaluator\n", arg[2]);
  check(smx_evaluator_create(arg[2], head.c_str(), &evaluator), "loading the model");
  check(smx_set_allow_fixed_workspace(evaluator, allow_fixed_workspace ? 1 : 0), "plan request");
  check(smx_set_execution_plan_request(evaluator, "direct", execution_profile.c_str(), debug_plan.c_str()),
        "plan request");
  // a MACEField model runs in the electric_field of the pair style
  // (pair_symmetrix_mace_kokkos.cpp:598-599); a plain model takes none
  int32_t field_model = 0;
  check(smx_has_field_coupling(evaluator, &field_model), "model info");
  if (field_model && !electric_field_set)
    error->all(FLERR, "MACEField models require pair_style symmetrix/mace/mi355x/kk electric_field Ex Ey Ez");
  if (electric_field_set) check(smx_set_electric_field(evaluator, electric_field, 3), "electric_field");
  SmxModelInfo info{};
  info.struct_size = sizeof(info);
  check(smx_evaluator_info(evaluator, &info), "model info");
  r_cut = info.r_cut;
  single_layer = info.num_interactions == 1;
  int64_t width = 0;
  check(smx_distributed_exchange(evaluator, 0, nullptr, nullptr, &width), "model info");
  row_floats = static_cast<int>(width);
  comm_forward = comm_reverse = single_layer ? 0 : row_floats;
  generation = 0;
  graph_nall = -1;
  std::vector<int32_t> numbers(info.num_elements);
  check(smx_evaluator_atomic_numbers(evaluator, numbers.data(), info.num_elements), "atomic numbers");

  // LAMMPS type t (1-based) -> model type of the element named for it
  const int ntypes = atom->ntypes;
  Kokkos::realloc(d_type_to_model, ntypes);
  auto h_map = Kokkos::create_mirror_view(d_type_to_model);
  for (int t = 0; t < ntypes; ++t) {
    const int z = element_number(arg[3 + t]);
    if (z == 0) error->all(FLERR, "pair_coeff: {} is not an element symbol", arg[3 + t]);
    h_map(t) = -1;
    for (int m = 0; m < info.num_elements; ++m)
      if (numbers[m] == z) h_map(t) = m;
    if (h_map(t) < 0) error->all(FLERR, "element {} is not in the MACE model", arg[3 + t]);
  }
  Kokkos::deep_copy(d_type_to_model, h_map);
  for (int i = 1; i <= ntypes; i++)
    for (int j = i; j <= ntypes; j++) setflag[i][j] = 1;
}

template <class DeviceType>
double PairSymmetrixMACEMI355X<DeviceType>::init_one(int i, int j)
{
  if (setflag[i][j] == 0) error->all(FLERR, "All pair coeffs are not set");
  return r_cut;
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::init_style()
{
  if (atom->map_user == atom->MAP_NONE)
    error->all(FLERR, "symmetrix/mace/mi355x/kk requires 'atom_modify map [yes|array|hash]'");
  if (force->newton_pair == 0) error->all(FLERR, "symmetrix/mace/mi355x/kk requires newton pair on");
  auto request = neighbor->add_request(this, NeighConst::REQ_FULL);
  request->set_kokkos_host(std::is_same_v<DeviceType, LMPHostType> && !std::is_same_v<DeviceType, LMPDeviceType>);
  request->set_kokkos_device(std::is_same_v<DeviceType, LMPDeviceType>);
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::compute(int eflag, int vflag)
{
  ev_init(eflag, vflag, 0);
  if (eflag_atom) {
    if (k_eatom.template view<DeviceType>().extent(0) < (size_t) maxeatom) {
      memoryKK->destroy_kokkos(k_eatom, eatom);
      memoryKK->create_kokkos(k_eatom, eatom, maxeatom, "pair:eatom");
    }
    Kokkos::deep_copy(k_eatom.template view<DeviceType>(), 0.0);
  }
  atomKK->sync(execution_space, X_MASK | F_MASK | TYPE_MASK | TAG_MASK);
  if (mode == "mpi_message_passing")
    compute_mpi_message_passing();
  else
    compute_no_domain_decomposition();
  if (eflag_atom) {
    k_eatom.template modify<DeviceType>();
    k_eatom.template sync<LMPHostType>();
  }
  if (eflag || vflag)
    atomKK->modified(execution_space, datamask_modify);
  else
    atomKK->modified(execution_space, F_MASK);
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::compute_no_domain_decomposition()
{
  auto x = atomKK->k_x.template view<DeviceType>();
  auto f = atomKK->k_f.template view<DeviceType>();
  auto type = atomKK->k_type.template view<DeviceType>();
  auto *k_list = static_cast<NeighListKokkos<DeviceType> *>(list);
  const int nall = atom->nlocal + atom->nghost;
  const bool rebuild = neighbor->ago == 0;

  // owner of every atom (atom->map(tag)), refreshed with the neighbour list
  if (rebuild || d_owner.extent(0) < (size_t) nall) {
    if (d_owner.extent(0) < (size_t) nall) {
      Kokkos::realloc(d_owner, nall);
      h_owner = Kokkos::create_mirror_view(d_owner);
    }
    for (int j = 0; j < nall; ++j) h_owner(j) = atom->map(atom->tag[j]);
    Kokkos::deep_copy(d_owner, h_owner);
  }

  SmxLammpsArgsV2 a{};
  a.struct_size = sizeof(a);
  a.inum = k_list->inum;
  a.nall = nall;
  a.ntypes = atom->ntypes;
  a.ilist = k_list->d_ilist.data();
  a.numneigh = k_list->d_numneigh.data();
  a.neighbors = k_list->d_neighbors.data();
  a.stride_atom = k_list->d_neighbors.stride(0);
  a.stride_neighbor = k_list->d_neighbors.stride(1);
  a.x = x.data();
  a.type = type.data();
  a.type_to_model = d_type_to_model.data();
  a.owner = d_owner.data();
  a.rebuild = rebuild ? 1 : 0;
  a.f = f.data();
  a.eatom = eflag_atom ? k_eatom.template view<DeviceType>().data() : nullptr;
  a.stream = DeviceType().hip_stream();
  double energy = 0.0, v[6] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
  check(smx_lammps_compute(evaluator, reinterpret_cast<const SmxLammpsArgsV1 *>(&a), &energy, v),
        "evaluation");

  if (eflag_global) eng_vdwl += energy;
  if (vflag_global)
    for (int k = 0; k < 6; ++k) virial[k] += v[k];
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::compute_mpi_message_passing()
{
  auto x = atomKK->k_x.template view<DeviceType>();
  auto f = atomKK->k_f.template view<DeviceType>();
  auto type = atomKK->k_type.template view<DeviceType>();
  auto *k_list = static_cast<NeighListKokkos<DeviceType> *>(list);
  auto d_ilist = k_list->d_ilist;
  auto d_numneigh = k_list->d_numneigh;
  auto d_neighbors = k_list->d_neighbors;
  const int inum = k_list->inum, nlocal = atom->nlocal, nall = nlocal + atom->nghost;
  if (inum != nlocal)
    error->all(FLERR, "symmetrix/mace/mi355x/kk mpi_message_passing requires one receiver for every owned atom");
  auto map = d_type_to_model;

  // the rank's feature graph on neighbour-list rebuilds (:1365-1475)
  if (neighbor->ago == 0 || generation == 0 || nall != graph_nall) {
    Kokkos::realloc(d_feature_types, nall);
    Kokkos::realloc(d_receiver_features, inum);
    Kokkos::realloc(d_node_types, inum);
    Kokkos::realloc(d_num_neigh, inum);
    Kokkos::realloc(d_first, inum + 1);
    auto ft = d_feature_types;
    auto rf = d_receiver_features;
    auto nt = d_node_types;
    auto nn = d_num_neigh;
    auto first = d_first;
    Kokkos::parallel_for(
        Kokkos::RangePolicy<DeviceType>(0, nall), KOKKOS_LAMBDA(const int i) { ft(i) = map(type(i) - 1); });
    Kokkos::parallel_for(
        Kokkos::RangePolicy<DeviceType>(0, inum), KOKKOS_LAMBDA(const int ii) {
          const int i = d_ilist(ii);
          rf(ii) = i;
          nt(ii) = map(type(i) - 1);
          nn(ii) = d_numneigh(i);
        });
    int64_t total = 0;
    Kokkos::parallel_scan(
        Kokkos::RangePolicy<DeviceType>(0, inum),
        KOKKOS_LAMBDA(const int ii, int64_t &sum, const bool final) {
          if (final) first(ii) = static_cast<int>(sum);
          sum += nn(ii);
        },
        total);
    if (total > INT_MAX) error->one(FLERR, "symmetrix/mace/mi355x/kk rank-local edge count exceeds INT_MAX");
    num_edges = total;
    Kokkos::realloc(d_neigh, num_edges > 0 ? num_edges : 1);
    Kokkos::realloc(d_neigh_types, num_edges > 0 ? num_edges : 1);
    auto nb = d_neigh;
    auto nbt = d_neigh_types;
    Kokkos::parallel_for(
        Kokkos::RangePolicy<DeviceType>(0, inum), KOKKOS_LAMBDA(const int ii) {
          const int i = d_ilist(ii);
          for (int jj = 0; jj < d_numneigh(i); ++jj) {
            const int j = d_neighbors(i, jj) & NEIGHMASK;
            nb(first(ii) + jj) = j;
            nbt(first(ii) + jj) = map(type(j) - 1);
          }
        });
    Kokkos::fence();
    check(smx_prepare_factorized_feature_graph_device(evaluator, inum, nall, d_receiver_features.data(),
                                                      d_node_types.data(), d_feature_types.data(),
                                                      d_num_neigh.data(), num_edges, d_neigh.data(),
                                                      d_neigh_types.data(), &generation),
          "feature graph");
    graph_nall = nall;
  }

  // the feature nodes' positions are x itself (local and ghost rows, by
  // LAMMPS index): the library forms each edge vector x[j] - x[i], scaled
  // to the cutoff when longer (prepared execution keeps every listed
  // neighbour, :1520-1560)
  Kokkos::fence();
  if (single_layer) {
    check(smx_compute_factorized_single_layer_distributed_positions_evaluation(evaluator, generation, inum, nall,
                                                                               x.data(), 1),
          "evaluation");
  } else {
    check(smx_begin_factorized_distributed_positions_evaluation(evaluator, generation, inum, nall, x.data(), 1),
          "evaluation (prefix)");
    // the receivers' H1 rows at their LAMMPS indices, then the ghosts' from
    // their owners (:1582-1689)
    float *rows = nullptr;
    int64_t nrows = 0, width = 0;
    check(smx_distributed_exchange(evaluator, 0, &rows, &nrows, &width), "H1 rows");
    Kokkos::realloc(d_h1, static_cast<size_t>(nall > 0 ? nall : 1) * row_floats);
    {
      auto h1 = d_h1;
      const size_t rfl = row_floats;
      Kokkos::parallel_for(
          Kokkos::RangePolicy<DeviceType>(0, static_cast<size_t>(inum) * rfl), KOKKOS_LAMBDA(const size_t q) {
            h1(static_cast<size_t>(d_ilist(q / rfl)) * rfl + q % rfl) = rows[q];
          });
    }
    Kokkos::fence();
    comm->forward_comm(this);
    Kokkos::fence();
    check(smx_continue_factorized_distributed_evaluation(evaluator, d_h1.data(), nall, 1), "evaluation (middle)");
    // the ghosts' H1 adjoints onto their owners (:1690-1704)
    check(smx_distributed_exchange(evaluator, 1, &exchange_rows, &nrows, &width), "H1 adjoint rows");
    comm->reverse_comm(this);
    Kokkos::fence();
    exchange_rows = nullptr;
    check(smx_finish_factorized_distributed_evaluation(evaluator, nullptr, 0, 1), "evaluation (suffix)");
  }

  // feature-node forces onto the local and ghost rows (the ghosts' then go
  // to their owners through LAMMPS's reverse communication), energies, virial
  double energy = 0.0, stress[9];
  check(smx_reduce_prepared_node_forces(evaluator, generation, nullptr), "forces");
  check(smx_reduce_prepared_stress(evaluator, generation, 1.0, stress), "virial");
  check(smx_total_energy_device(evaluator, &energy), "energy");
  check(smx_synchronize(evaluator), "synchronize");
  SmxDeviceOutputs o{};
  o.struct_size = sizeof(o);
  check(smx_device_outputs(evaluator, &o), "outputs");
  const double *af = o.atom_forces, *ne = o.node_energies;
  Kokkos::parallel_for(
      Kokkos::RangePolicy<DeviceType>(0, nall), KOKKOS_LAMBDA(const int i) {
        f(i, 0) += af[3 * i];
        f(i, 1) += af[3 * i + 1];
        f(i, 2) += af[3 * i + 2];
      });
  if (eflag_atom) {
    auto eatom_d = k_eatom.template view<DeviceType>();
    Kokkos::parallel_for(
        Kokkos::RangePolicy<DeviceType>(0, inum), KOKKOS_LAMBDA(const int ii) { eatom_d(d_ilist(ii)) += ne[ii]; });
  }
  Kokkos::fence();
  // with unit volume the stress is minus the virial sum over the rank's
  // edges; a rank's partial sum is not symmetric, so each off-diagonal pair
  // is averaged as in the no_domain_decomposition mode
  if (eflag_global) eng_vdwl += energy;
  if (vflag_global) {
    virial[0] -= stress[0];
    virial[1] -= stress[4];
    virial[2] -= stress[8];
    virial[3] -= 0.5 * (stress[1] + stress[3]);
    virial[4] -= 0.5 * (stress[2] + stress[6]);
    virial[5] -= 0.5 * (stress[5] + stress[7]);
  }
}

// ------------------------------------------------------------ communication
// Forward: H1 rows of the atoms in the send list into the buffer, and the
// received rows into the ghost rows first..first+n.  Reverse: the ghosts'
// H1 adjoint rows into the buffer, and the received rows added onto the
// owners in the list (pair_symmetrix_mace_kokkos.cpp:738-1008).
template <class DeviceType>
int PairSymmetrixMACEMI355X<DeviceType>::pack_forward_comm_kokkos(int n, DAT::tdual_int_1d k_sendlist,
                                                                  DAT::tdual_double_1d &buf, int, int *)
{
  auto list = k_sendlist.template view<DeviceType>();
  auto b = buf.template view<DeviceType>();
  auto h1 = d_h1;
  const size_t rfl = row_floats;
  Kokkos::parallel_for(
      Kokkos::RangePolicy<DeviceType>(0, static_cast<size_t>(n) * rfl), KOKKOS_LAMBDA(const size_t q) {
        b(q) = h1(static_cast<size_t>(list(q / rfl)) * rfl + q % rfl);
      });
  return n * row_floats;
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::unpack_forward_comm_kokkos(int n, int first, DAT::tdual_double_1d &buf)
{
  auto b = buf.template view<DeviceType>();
  auto h1 = d_h1;
  const size_t rfl = row_floats, base = static_cast<size_t>(first) * rfl;
  Kokkos::parallel_for(
      Kokkos::RangePolicy<DeviceType>(0, static_cast<size_t>(n) * rfl),
      KOKKOS_LAMBDA(const size_t q) { h1(base + q) = static_cast<float>(b(q)); });
}

template <class DeviceType>
int PairSymmetrixMACEMI355X<DeviceType>::pack_reverse_comm_kokkos(int n, int first, DAT::tdual_double_1d &buf)
{
  auto b = buf.template view<DeviceType>();
  const float *rows = exchange_rows;
  const size_t rfl = row_floats, base = static_cast<size_t>(first) * rfl;
  Kokkos::parallel_for(
      Kokkos::RangePolicy<DeviceType>(0, static_cast<size_t>(n) * rfl),
      KOKKOS_LAMBDA(const size_t q) { b(q) = rows[base + q]; });
  return n * row_floats;
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::unpack_reverse_comm_kokkos(int n, DAT::tdual_int_1d k_sendlist,
                                                                     DAT::tdual_double_1d &buf)
{
  auto list = k_sendlist.template view<DeviceType>();
  auto b = buf.template view<DeviceType>();
  float *rows = exchange_rows;
  const size_t rfl = row_floats;
  Kokkos::parallel_for(
      Kokkos::RangePolicy<DeviceType>(0, static_cast<size_t>(n) * rfl), KOKKOS_LAMBDA(const size_t q) {
        Kokkos::atomic_add(&rows[static_cast<size_t>(list(q / rfl)) * rfl + q % rfl], static_cast<float>(b(q)));
      });
}

// host-buffer forms: the same packing through a device staging buffer
template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::stage(size_t values)
{
  if (d_stage.extent(0) < values) Kokkos::realloc(d_stage, values);
}

template <class DeviceType>
int PairSymmetrixMACEMI355X<DeviceType>::pack_forward_comm(int n, int *list, double *buf, int, int *)
{
  const size_t rfl = row_floats, values = static_cast<size_t>(n) * rfl;
  stage(values);
  if (d_stage_list.extent(0) < static_cast<size_t>(n)) Kokkos::realloc(d_stage_list, n);
  Kokkos::deep_copy(Kokkos::subview(d_stage_list, std::make_pair(0, n)),
                    Kokkos::View<const int *, Kokkos::HostSpace, Kokkos::MemoryTraits<Kokkos::Unmanaged>>(list, n));
  auto l = d_stage_list;
  auto b = d_stage;
  auto h1 = d_h1;
  Kokkos::parallel_for(
      Kokkos::RangePolicy<DeviceType>(0, values),
      KOKKOS_LAMBDA(const size_t q) { b(q) = h1(static_cast<size_t>(l(q / rfl)) * rfl + q % rfl); });
  Kokkos::deep_copy(Kokkos::View<double *, Kokkos::HostSpace, Kokkos::MemoryTraits<Kokkos::Unmanaged>>(buf, values),
                    Kokkos::subview(d_stage, std::make_pair(size_t(0), values)));
  return n * row_floats;
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::unpack_forward_comm(int n, int first, double *buf)
{
  const size_t rfl = row_floats, values = static_cast<size_t>(n) * rfl, base = static_cast<size_t>(first) * rfl;
  stage(values);
  Kokkos::deep_copy(Kokkos::subview(d_stage, std::make_pair(size_t(0), values)),
                    Kokkos::View<const double *, Kokkos::HostSpace, Kokkos::MemoryTraits<Kokkos::Unmanaged>>(
                        buf, values));
  auto b = d_stage;
  auto h1 = d_h1;
  Kokkos::parallel_for(
      Kokkos::RangePolicy<DeviceType>(0, values),
      KOKKOS_LAMBDA(const size_t q) { h1(base + q) = static_cast<float>(b(q)); });
}

template <class DeviceType>
int PairSymmetrixMACEMI355X<DeviceType>::pack_reverse_comm(int n, int first, double *buf)
{
  const size_t rfl = row_floats, values = static_cast<size_t>(n) * rfl, base = static_cast<size_t>(first) * rfl;
  stage(values);
  auto b = d_stage;
  const float *rows = exchange_rows;
  Kokkos::parallel_for(
      Kokkos::RangePolicy<DeviceType>(0, values), KOKKOS_LAMBDA(const size_t q) { b(q) = rows[base + q]; });
  Kokkos::deep_copy(Kokkos::View<double *, Kokkos::HostSpace, Kokkos::MemoryTraits<Kokkos::Unmanaged>>(buf, values),
                    Kokkos::subview(d_stage, std::make_pair(size_t(0), values)));
  return n * row_floats;
}

template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::unpack_reverse_comm(int n, int *list, double *buf)
{
  const size_t rfl = row_floats, values = static_cast<size_t>(n) * rfl;
  stage(values);
  if (d_stage_list.extent(0) < static_cast<size_t>(n)) Kokkos::realloc(d_stage_list, n);
  Kokkos::deep_copy(Kokkos::subview(d_stage_list, std::make_pair(0, n)),
                    Kokkos::View<const int *, Kokkos::HostSpace, Kokkos::MemoryTraits<Kokkos::Unmanaged>>(list, n));
  Kokkos::deep_copy(Kokkos::subview(d_stage, std::make_pair(size_t(0), values)),
                    Kokkos::View<const double *, Kokkos::HostSpace, Kokkos::MemoryTraits<Kokkos::Unmanaged>>(
                        buf, values));
  auto l = d_stage_list;
  auto b = d_stage;
  float *rows = exchange_rows;
  Kokkos::parallel_for(
      Kokkos::RangePolicy<DeviceType>(0, values), KOKKOS_LAMBDA(const size_t q) {
        Kokkos::atomic_add(&rows[static_cast<size_t>(l(q / rfl)) * rfl + q % rfl], static_cast<float>(b(q)));
      });
}

namespace LAMMPS_NS {
template class PairSymmetrixMACEMI355X<LMPDeviceType>;
}
