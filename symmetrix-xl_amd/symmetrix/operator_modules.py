"""M0 / R0 operator modules: the reference's code-object container for its
product-basis and first-interaction radial operators, built from this
project's gfx950 kernels (include/symmetrix_operator_modules.h,
csrc/operator_module.hip).

The reference loads such a module with ``OperatorModule::load``
(libsymmetrix/source/jit_operator_module.cpp:236-373): it reads a raw ELF64
code object, checks the ``symmetrix_operator_*_v1`` identity symbols against
what the model expects and launches the ``symmetrix_m0_*_v1`` /
``symmetrix_r0_*_v1`` kernels with one argument packet by value on
min(ceil(work / threads), persistent_blocks) blocks.

This module provides
  * the argument packets as ctypes structures (byte layouts of
    jit_operator_module_abi.h:23-79: 80, 40 and 256 bytes);
  * builders that render a module for a contract -- the reference's own
    operator metadata (``jit_m0_device_metadata`` / ``jit_r0_device_metadata``
    of jit_operator_codegen.py:40-84, 584-615: identity strings, channels,
    monomial groups) -- and compile it with hipcc into a code object;
  * a loader with the reference loader's checks and launch rule, used by the
    tests in place of the reference's C++ loader.
"""

import ctypes
import os
import subprocess
import tempfile

_HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.normpath(os.path.join(_HERE, "..", "csrc"))
MODULE_DIR = os.path.join(_HERE, "modules")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

KIND_M0, KIND_R0 = 1, 2
THREADS = 256
M0_CAPABILITIES = 0x1F
R0_CAPABILITIES = 0x7F00
M0_KERNELS = ("symmetrix_m0_forward_v1", "symmetrix_m0_reverse_v1")
R0_KERNELS = ("symmetrix_r0_density_prepare_v1", "symmetrix_r0_forward_v1", "symmetrix_r0_reverse_prepare_v1",
              "symmetrix_r0_coordinate_reverse_v1")


class M0Args(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("reserved", ctypes.c_uint32), ("num_nodes", ctypes.c_int64),
                ("channels", ctypes.c_int32), ("capture_input_scale_adjoint", ctypes.c_int32),
                ("node_types", ctypes.c_void_p), ("input", ctypes.c_void_p), ("weights", ctypes.c_void_p),
                ("output_adjoint", ctypes.c_void_p), ("output", ctypes.c_void_p), ("input_adjoint", ctypes.c_void_p),
                ("input_scale_adjoint", ctypes.c_void_p)]


class R0Spline(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("edge_types", ctypes.c_uint32), ("intervals", ctypes.c_uint32),
                ("functions", ctypes.c_uint32), ("h", ctypes.c_double), ("x0", ctypes.c_double),
                ("coefficients", ctypes.c_void_p)]


class R0Args(ctypes.Structure):
    _fields_ = [("struct_size", ctypes.c_uint32), ("receiver_base", ctypes.c_uint32), ("num_nodes", ctypes.c_int64),
                ("num_edges", ctypes.c_int64), ("active_type_count", ctypes.c_int32), ("channels", ctypes.c_int32),
                ("l_max", ctypes.c_int32), ("coordinates_are_unit", ctypes.c_int32),
                ("apply_density_scale", ctypes.c_int32), ("use_precomputed_scale_adjoint", ctypes.c_int32),
                ("node_types", ctypes.c_void_p), ("num_neigh", ctypes.c_void_p), ("first_neigh", ctypes.c_void_p),
                ("neigh_types", ctypes.c_void_p), ("edge_receivers", ctypes.c_void_p),
                ("type_to_active", ctypes.c_void_p), ("coordinates", ctypes.c_void_p), ("radius", ctypes.c_void_p),
                ("radial", R0Spline), ("density", R0Spline), ("harmonics", ctypes.c_void_p),
                ("harmonic_gradients", ctypes.c_void_p), ("output", ctypes.c_void_p),
                ("output_adjoint", ctypes.c_void_p), ("density_state", ctypes.c_void_p),
                ("precomputed_scale_adjoint", ctypes.c_void_p), ("directed_forces", ctypes.c_void_p),
                ("cutoff", ctypes.c_double)]


def spline(coefficients=None, edge_types=0, intervals=0, functions=0, h=0.0, x0=0.0):
    return R0Spline(ctypes.sizeof(R0Spline), edge_types, intervals, functions, h, x0, coefficients)


# ----------------------------------------------------------------------- build
def compiled_module_path(kind, channels, l_max, L_max=None, correlation=None):
    """Path of a module the Makefile builds for a compiled shape (test
    identities: artifact ``symmetrix-mi355x-<name>``, structure
    ``compiled:<name>``, target gfx950)."""
    if kind == KIND_M0:
        name = "m0_c%d_l%d_L%d_k%d" % (channels, l_max, L_max, correlation)
    else:
        name = "r0_c%d_l%d" % (channels, l_max)
    return os.path.join(MODULE_DIR, name + ".co"), name


def _c_string(text):
    text = str(text)
    if not text or len(text.encode()) >= 511 or any(c in text for c in '"\\\n'):
        raise ValueError("identity strings must be non-empty printable text under 511 bytes without quotes")
    return '"%s"' % text


def pack_monomial(components):
    """Packed monomial (variables in bytes 0..2 in the given order, degree in
    byte 3), the product order of the reference's generated code."""
    comps = [int(c) for c in components]
    if not 1 <= len(comps) <= 3 or any(not 0 <= c < 256 for c in comps):
        raise ValueError("monomials of degree 1..3 over at most 256 variables are supported")
    p = len(comps) << 24
    for i, c in enumerate(comps):
        p |= c << (8 * i)
    return p


def render_m0_source(terms, offsets, channels, l_max, correlation, artifact_id, structure_fingerprint,
                     target="gfx950"):
    """Wrapper source of an M0 module: the monomial table (packed terms,
    per-output offsets) and identity, then the shared module source."""
    n_out = len(offsets) - 1
    lines = [
        "// Rendered by symmetrix.operator_modules: M0 operator module.",
        "#include <array>",
        "#include <cstdint>",
        "struct ContractTable {",
        "    static constexpr bool available = true;",
        "    static constexpr int NOUT = %d;" % n_out,
        "    static constexpr int NT = %d;" % len(terms),
        "    static constexpr std::array<int, NOUT + 1> offset = {%s};" % ", ".join(str(int(o)) for o in offsets),
        "    static constexpr std::array<std::int32_t, NT> terms = {%s};" % ", ".join(
            "0x%08x" % int(t) for t in terms),
        "};",
        "#define SMX_OPMOD_KIND 1",
        "#define SMX_OPMOD_CHANNELS %d" % int(channels),
        "#define SMX_OPMOD_LMAX %d" % int(l_max),
        "#define SMX_OPMOD_CORRELATION %d" % int(correlation),
        "#define SMX_OPMOD_TABLE ContractTable",
        "#define SMX_OPMOD_ARTIFACT %s" % _c_string(artifact_id),
        "#define SMX_OPMOD_STRUCTURE %s" % _c_string(structure_fingerprint),
        "#define SMX_OPMOD_TARGET %s" % _c_string(target),
        '#include "operator_module.hip"',
        "",
    ]
    return "\n".join(lines)


def render_r0_source(channels, l_max, artifact_id, structure_fingerprint, target="gfx950"):
    """Wrapper source of a scalar-source R0 module."""
    if int(channels) > THREADS or THREADS % int(channels):
        raise ValueError("R0 modules need channels dividing %d" % THREADS)
    return "\n".join([
        "// Rendered by symmetrix.operator_modules: R0 operator module.",
        "#define SMX_OPMOD_KIND 2",
        "#define SMX_OPMOD_CHANNELS %d" % int(channels),
        "#define SMX_OPMOD_LMAX %d" % int(l_max),
        "#define SMX_OPMOD_ARTIFACT %s" % _c_string(artifact_id),
        "#define SMX_OPMOD_STRUCTURE %s" % _c_string(structure_fingerprint),
        "#define SMX_OPMOD_TARGET %s" % _c_string(target),
        '#include "operator_module.hip"',
        "",
    ])


def compile_module(source, out_path):
    """Compile a rendered wrapper into a raw gfx950 ELF code object."""
    os.makedirs(os.path.dirname(os.path.abspath(out_path)) or ".", exist_ok=True)
    with tempfile.TemporaryDirectory() as tmp:
        src = os.path.join(tmp, "module.hip")
        with open(src, "w") as f:
            f.write(source)
        cmd = [HIPCC, "--cuda-device-only", "--no-gpu-bundle-output", "--offload-arch=gfx950", "-O3", "-std=c++20",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument",
               "-I", CSRC, src, "-o", out_path]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError("module compilation failed:\n" + r.stderr[-4000:])
    return out_path


def build_m0_module(metadata, out_path):
    """Build an M0 module from the reference's M0 operator metadata (the dict
    ``jit_m0_device_metadata`` returns: artifact_id, structure_fingerprint,
    target, correlation and the normalised contract with ``channels`` and
    ``monomial_groups`` [{output_component, terms: [[v, ...], ...]}, ...])."""
    contract = metadata["contract"]
    if metadata.get("precision", "float32") != "float32":
        raise ValueError("this build's operator modules are FP32")
    groups = sorted(contract["monomial_groups"], key=lambda g: int(g["output_component"]))
    terms, offsets = [], [0]
    for g in groups:
        terms += [pack_monomial(t) for t in g["terms"]]
        offsets.append(len(terms))
    n_in = int(metadata["input_components"])
    l_max = int(round(n_in ** 0.5)) - 1
    if (l_max + 1) ** 2 != n_in:
        raise ValueError("M0 input components must be (l_max+1)^2")
    src = render_m0_source(terms, offsets, contract["channels"], l_max, metadata["correlation"],
                           metadata["artifact_id"], metadata["structure_fingerprint"], metadata.get("target", "gfx950"))
    return compile_module(src, out_path)


def build_r0_module(metadata, out_path):
    """Build an R0 module from the reference's R0 operator metadata (the dict
    ``jit_r0_device_metadata`` returns)."""
    if metadata.get("precision", "float32") != "float32":
        raise ValueError("this build's operator modules are FP32")
    n = int(metadata["input_components"])
    l_max = int(round(n ** 0.5)) - 1
    src = render_r0_source(metadata["contract"]["channels"], l_max, metadata["artifact_id"],
                           metadata["structure_fingerprint"], metadata.get("target", "gfx950"))
    return compile_module(src, out_path)


# ---------------------------------------------------------------------- load
def read_code_object(path):
    """The module bytes, checked as the reference's loader checks them
    (little-endian ELF64, jit_device_plugin_common.hpp:71-82)."""
    with open(path, "rb") as f:
        data = f.read()
    if len(data) < 64 or data[:4] != b"\x7fELF" or data[4] != 2 or data[5] != 1:
        raise ValueError("%s is not a little-endian ELF64 code object" % path)
    return data


_hip = None


def _hip_lib():
    global _hip
    if _hip is None:
        h = ctypes.CDLL("libamdhip64.so")
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        h.hipModuleLoadData.argtypes = [ctypes.POINTER(vp), ctypes.c_char_p]
        h.hipModuleUnload.argtypes = [vp]
        h.hipModuleGetFunction.argtypes = [ctypes.POINTER(vp), vp, ctypes.c_char_p]
        h.hipModuleGetGlobal.argtypes = [ctypes.POINTER(vp), ctypes.POINTER(sz), vp, ctypes.c_char_p]
        h.hipMemcpyDtoH.argtypes = [vp, vp, sz]
        h.hipModuleLaunchKernel.argtypes = [vp, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                                            ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, vp,
                                            ctypes.POINTER(vp), ctypes.POINTER(vp)]
        _hip = h
    return _hip


class CodeObject:
    """A loaded operator module: identity values and kernel handles."""

    def __init__(self, path):
        h = _hip_lib()
        self._data = read_code_object(path)
        self.module = ctypes.c_void_p()
        rc = h.hipModuleLoadData(ctypes.byref(self.module), self._data)
        if rc != 0:
            raise RuntimeError("hipModuleLoadData failed (%d) for %s" % (rc, path))
        self.identity = {}
        for name, kind in (("abi_version", "u32"), ("kind", "u32"), ("scalar_kind", "u32"), ("scalar_size", "u32"),
                           ("capabilities", "u32"), ("input_components", "i32"), ("output_components", "i32"),
                           ("correlation", "i32"), ("term_count", "i32"), ("threads", "i32"),
                           ("artifact_id", "str"), ("structure_fingerprint", "str"), ("target", "str")):
            self.identity[name] = self._global("symmetrix_operator_%s_v1" % name, kind)
        names = M0_KERNELS if self.identity["kind"] == KIND_M0 else R0_KERNELS
        self.functions = {}
        for n in names:
            f = ctypes.c_void_p()
            rc = h.hipModuleGetFunction(ctypes.byref(f), self.module, n.encode())
            if rc != 0:
                raise RuntimeError("module has no kernel %s (%d)" % (n, rc))
            self.functions[n] = f

    def _global(self, symbol, kind):
        h = _hip_lib()
        ptr, size = ctypes.c_void_p(), ctypes.c_size_t()
        rc = h.hipModuleGetGlobal(ctypes.byref(ptr), ctypes.byref(size), self.module, symbol.encode())
        if rc != 0:
            raise RuntimeError("missing identity symbol %s" % symbol)
        buf = ctypes.create_string_buffer(size.value)
        if h.hipMemcpyDtoH(buf, ptr, size) != 0:
            raise RuntimeError("hipMemcpyDtoH failed for %s" % symbol)
        raw = buf.raw
        if kind == "u32":
            return int.from_bytes(raw[:4], "little")
        if kind == "i32":
            return int.from_bytes(raw[:4], "little", signed=True)
        if not raw.endswith(b"\0"):
            raise RuntimeError("unterminated identity text %s" % symbol)
        return raw[:-1].decode()

    def launch(self, kernel, args, work_items, persistent_blocks, stream=None):
        """Launch as the reference's loader does: min(ceil(work/threads),
        persistent_blocks) blocks of the module's thread count; returns the
        hipError_t (0 on success).  Nothing is launched for no work."""
        if work_items == 0:
            return 0
        threads = self.identity["threads"]
        blocks = min(-(-int(work_items) // threads), int(persistent_blocks))
        params = (ctypes.c_void_p * 1)(ctypes.cast(ctypes.byref(args), ctypes.c_void_p))
        return _hip_lib().hipModuleLaunchKernel(self.functions[kernel], blocks, 1, 1, threads, 1, 1, 0, stream,
                                                params, None)

    def __del__(self):
        if getattr(self, "module", None):
            _hip_lib().hipModuleUnload(self.module)
            self.module = ctypes.c_void_p()
