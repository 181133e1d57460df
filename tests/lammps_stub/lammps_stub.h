// Stand-ins for the parts of the LAMMPS (KOKKOS package) and Kokkos APIs that
// the pair style symmetrix/mace/mi355x/kk uses, with their public signatures,
// so that the class can be type-checked (g++ -fsyntax-only) where LAMMPS and
// Kokkos are not installed.  Test infrastructure: nothing here runs, and the
// library's own header (include/symmetrix_mi355x.h) is the real one.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <type_traits>
#include <utility>

struct ihipStream_t;
typedef ihipStream_t* hipStream_t;

// ---------------------------------------------------------------- Kokkos
namespace Kokkos {

struct HostSpace;
struct Serial {
  using memory_space = HostSpace;
};
struct HIPSpace;
struct HIP {
  using memory_space = HIPSpace;
  hipStream_t hip_stream() const { return nullptr; }
};
struct HostSpace {
  using execution_space = Serial;
};
struct LayoutRight {};
enum MemoryTraitsFlags : unsigned { Unmanaged = 0x01, Atomic = 0x02 };
template <unsigned T>
struct MemoryTraits {};

namespace stub {
// value type and rank of a View data type: T*, T**, T*[N]
template <class T>
struct data_of {
  using value = T;
  static constexpr int rank = 0;
};
template <class T>
struct data_of<T*> {
  using value = typename data_of<T>::value;
  static constexpr int rank = data_of<T>::rank + 1;
};
template <class T, std::size_t N>
struct data_of<T[N]> {
  using value = typename data_of<T>::value;
  static constexpr int rank = data_of<T>::rank + 1;
};
}  // namespace stub

template <class DataType, class... Properties>
class View {
 public:
  using value_type = typename stub::data_of<DataType>::value;
  using pointer_type = value_type*;
  using reference_type = value_type&;
  using HostMirror = View<DataType, HostSpace>;
  static constexpr int rank = stub::data_of<DataType>::rank;

  View() = default;
  explicit View(const std::string& label, std::size_t n0 = 0, std::size_t n1 = 0);
  View(pointer_type unmanaged, std::size_t n0, std::size_t n1 = 0);
  template <class D, class... P>
  View(const View<D, P...>& other);

  std::size_t extent(int dim) const;
  std::size_t stride(int dim) const;
  std::size_t size() const;
  pointer_type data() const;
  template <class I0>
  reference_type operator()(I0 i0) const;
  template <class I0, class I1>
  reference_type operator()(I0 i0, I1 i1) const;
};

template <class DataType, class... Properties>
typename View<DataType, Properties...>::HostMirror create_mirror_view(const View<DataType, Properties...>&);
template <class D1, class... P1, class D2, class... P2>
void deep_copy(const View<D1, P1...>& dst, const View<D2, P2...>& src);
template <class D, class... P>
void deep_copy(const View<D, P...>& dst, const typename View<D, P...>::value_type& value);
template <class D, class... P>
void realloc(View<D, P...>& v, std::size_t n0, std::size_t n1 = 0);
template <class D, class... P, class I>
View<D, P...> subview(const View<D, P...>& v, std::pair<I, I> range);

template <class DataType, class Layout, class Device>
class DualView {
 public:
  template <class Space>
  View<DataType, Device> view() const;
  template <class Space>
  void modify();
  template <class Space>
  void sync();
};

template <class ExecSpace>
struct RangePolicy {
  using index_type = std::int64_t;
  template <class B, class E>
  RangePolicy(B begin, E end);
};
// the bodies only state how the functors are called: f(i) and f(i, partial, final)
template <class Policy, class Functor>
void parallel_for(const Policy&, const Functor& f) {
  f(typename Policy::index_type(0));
}
template <class Policy, class Functor, class Result>
void parallel_scan(const Policy&, const Functor& f, Result& total) {
  f(typename Policy::index_type(0), total, true);
}
void fence();
template <class T>
void atomic_add(T* dst, T value);

}  // namespace Kokkos

#define KOKKOS_LAMBDA [=]
#define KOKKOS_INLINE_FUNCTION inline

// ---------------------------------------------------------------- LAMMPS
#define FLERR __FILE__, __LINE__
#define X_MASK 0x00000001
#define V_MASK 0x00000002
#define F_MASK 0x00000004
#define TAG_MASK 0x00000008
#define TYPE_MASK 0x00000010
#define ENERGY_MASK 0x00010000
#define VIRIAL_MASK 0x00020000

typedef Kokkos::HIP LMPDeviceType;
typedef Kokkos::Serial LMPHostType;

namespace LAMMPS_NS {

typedef int tagint;
#define NEIGHMASK 0x1FFFFFFF

enum ExecutionSpace { Host, Device };
template <class DeviceType>
struct ExecutionSpaceFromDevice {
  static constexpr ExecutionSpace space = std::is_same_v<DeviceType, LMPHostType> ? Host : Device;
};

template <class DeviceType>
struct ArrayTypes {};
struct DAT {
  typedef Kokkos::DualView<int*, Kokkos::LayoutRight, LMPDeviceType> tdual_int_1d;
  typedef Kokkos::DualView<double*, Kokkos::LayoutRight, LMPDeviceType> tdual_double_1d;
  typedef Kokkos::DualView<double*, Kokkos::LayoutRight, LMPDeviceType> tdual_efloat_1d;
  typedef Kokkos::DualView<double* [3], Kokkos::LayoutRight, LMPDeviceType> tdual_x_array;
  typedef Kokkos::DualView<double* [3], Kokkos::LayoutRight, LMPDeviceType> tdual_f_array;
};

class LAMMPS;
class Pair;

class Error {
 public:
  template <typename... Args>
  [[noreturn]] void all(const std::string& file, int line, const std::string& format, Args&&... args);
  template <typename... Args>
  [[noreturn]] void one(const std::string& file, int line, const std::string& format, Args&&... args);
  template <typename... Args>
  void warning(const std::string& file, int line, const std::string& format, Args&&... args);
};

class Memory {
 public:
  template <typename TYPE>
  TYPE** create(TYPE**& array, int n1, int n2, const char* name);
  template <typename TYPE>
  void destroy(TYPE**& array);
};

class MemoryKokkos : public Memory {
 public:
  template <typename TYPE>
  TYPE create_kokkos(TYPE& data, typename TYPE::value_type*& array, int n1, const char* name);
  template <class TYPE>
  TYPE create_kokkos(TYPE& data, double*& array, int n1, const char* name);
  template <class TYPE>
  void destroy_kokkos(TYPE& data, double* array);
};

class Atom {
 public:
  enum { MAP_NONE = 0, MAP_ARRAY = 1, MAP_HASH = 2, MAP_YES = 3 };
  int ntypes = 0, nlocal = 0, nghost = 0;
  tagint* tag = nullptr;
  int map_user = MAP_NONE;
  int map(tagint global) const;
};

class AtomKokkos : public Atom {
 public:
  DAT::tdual_x_array k_x;
  DAT::tdual_f_array k_f;
  DAT::tdual_int_1d k_type;
  void sync(ExecutionSpace space, unsigned int mask);
  void modified(ExecutionSpace space, unsigned int mask);
};

class Comm {
 public:
  int me = 0, nprocs = 1;
  void forward_comm(Pair* pair, int size = 0);
  void reverse_comm(Pair* pair, int size = 0);
};

class Force {
 public:
  int newton_pair = 1;
};

class NeighRequest {
 public:
  void set_kokkos_host(int flag);
  void set_kokkos_device(int flag);
};
namespace NeighConst {
enum { REQ_DEFAULT = 0, REQ_FULL = 1 << 0, REQ_GHOST = 1 << 1 };
}
class Neighbor {
 public:
  int ago = 0;
  NeighRequest* add_request(Pair* requestor, int flags = 0);
};

class NeighList {
 public:
  int inum = 0, gnum = 0;
};
template <class DeviceType>
class NeighListKokkos : public NeighList {
 public:
  Kokkos::View<int*, DeviceType> d_ilist, d_numneigh;
  Kokkos::View<int**, DeviceType> d_neighbors;
};

namespace utils {
template <typename... Args>
void logmesg(LAMMPS* lmp, const std::string& format, Args&&... args);
}

class Pointers {
 public:
  explicit Pointers(LAMMPS* ptr);
  virtual ~Pointers() = default;

 protected:
  LAMMPS* lmp;
  Memory* memory;
  Error* error;
  Atom* atom;
  Force* force;
  Comm* comm;
  Neighbor* neighbor;
  AtomKokkos* atomKK;
  MemoryKokkos* memoryKK;
};

class Pair : protected Pointers {
 public:
  explicit Pair(LAMMPS* lmp);
  ~Pair() override = default;

  double eng_vdwl = 0.0, eng_coul = 0.0;
  double virial[6] = {};
  double* eatom = nullptr;
  double** cutsq = nullptr;
  int** setflag = nullptr;
  int comm_forward = 0, comm_reverse = 0, comm_reverse_off = 0;
  int respa_enable = 0, one_coeff = 0, manybody_flag = 0, no_virial_fdotr_compute = 0;
  int reverse_comm_device = 0, kokkosable = 0;
  int allocated = 0, copymode = 0;
  int eflag_either = 0, eflag_global = 0, eflag_atom = 0, vflag_either = 0, vflag_global = 0;
  int maxeatom = 0;
  NeighList* list = nullptr;
  ExecutionSpace execution_space = Host;
  unsigned int datamask_read = 0, datamask_modify = 0;

  virtual void compute(int, int) = 0;
  virtual void settings(int, char**) = 0;
  virtual void coeff(int, char**) = 0;
  virtual double init_one(int, int);
  virtual void init_style();
  virtual int pack_forward_comm(int, int*, double*, int, int*) { return 0; }
  virtual void unpack_forward_comm(int, int, double*) {}
  virtual int pack_reverse_comm(int, int, double*) { return 0; }
  virtual void unpack_reverse_comm(int, int*, double*) {}

 protected:
  void ev_init(int eflag, int vflag, int alloc = 1);
};

class KokkosBase {
 public:
  KokkosBase() = default;
  virtual ~KokkosBase() = default;
  virtual int pack_forward_comm_kokkos(int, DAT::tdual_int_1d, DAT::tdual_double_1d&, int, int*) { return 0; }
  virtual void unpack_forward_comm_kokkos(int, int, DAT::tdual_double_1d&) {}
  virtual int pack_reverse_comm_kokkos(int, int, DAT::tdual_double_1d&) { return 0; }
  virtual void unpack_reverse_comm_kokkos(int, DAT::tdual_int_1d, DAT::tdual_double_1d&) {}
};

}  // namespace LAMMPS_NS
