/* ----------------------------------------------------------------------
   pair_style symmetrix/mace/mi355x/kk (see pair_symmetrix_mace_mi355x.h)

   compute() follows the reference's no-domain-decomposition path
   (pair_symmetrix_mace_kokkos.cpp:1010-1282) with the work inside
   smx_lammps_compute: graph on rebuilds, edge vectors from x, model,
   deterministic force gather onto local and ghost rows, per-atom energies and
   the virial.  The call is ordered after the work Kokkos queued on the
   execution space's stream (SmxLammpsArgsV2.stream).
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
// this build has them: the mode token (only no_domain_decomposition),
// profile capacity|speed and its low_memory yes|no alias, allow_fixed_workspace
// yes|no, head NAME, streamed_edges auto|direct, _debug_execution_plan ID,
// electric_field Ex Ey Ez (MACEField, :207-224).  The JIT artefact keywords
// name files this build does not load (warned and skipped); the
// message-passing modes are refused.
template <class DeviceType>
void PairSymmetrixMACEMI355X<DeviceType>::settings(int narg, char **arg)
{
  if (comm->nprocs != 1)
    error->all(FLERR, "pair_style symmetrix/mace/mi355x/kk runs on one MPI rank (no_domain_decomposition)");
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
    if (key == "no_domain_decomposition") {
      continue;
    } else if (key == "mpi_message_passing" || key == "no_mpi_message_passing") {
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
  if (eflag_atom) {
    k_eatom.template modify<DeviceType>();
    k_eatom.template sync<LMPHostType>();
  }
  if (eflag || vflag)
    atomKK->modified(execution_space, datamask_modify);
  else
    atomKK->modified(execution_space, F_MASK);
}

namespace LAMMPS_NS {
template class PairSymmetrixMACEMI355X<LMPDeviceType>;
}
