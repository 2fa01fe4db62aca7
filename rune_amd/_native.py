"""ctypes binding of ``librune_hip.so`` (the C ABI in ``include/rune_hip.h``).

The library is built in-tree by ``__graft_entry__.build()`` (or ``make -C
rune_amd/csrc``).  There is no fallback: if the library is missing or no HIP
device is visible, every entry point raises.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "csrc" / "librune_hip.so"

RUNE_OK, ERR_ARGUMENT, ERR_HIP, ERR_OVERFLOW, ERR_TYPE, ERR_STATE = range(6)
FAMILY_MOBIUS, FAMILY_NEP = 0, 1
ACT = {"tanh": 0, "silu": 1, "swish": 1, "gelu": 2}
ZBL_NONE, ZBL_UNIVERSAL, ZBL_FLEXIBLE = 0, 1, 2


class NativeError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


class ModelConfig(C.Structure):
    _fields_ = [
        ("family", C.c_int32), ("n_types", C.c_int32),
        ("n_desc_radial", C.c_int32), ("k_radial", C.c_int32),
        ("n_desc_angular", C.c_int32), ("k_angular", C.c_int32),
        ("l_max", C.c_int32), ("has_q", C.c_int32 * 6),
        ("rc_radial", C.c_double), ("rc_angular", C.c_double),
        ("hidden_dim", C.c_int32), ("ffn_dim", C.c_int32), ("blocks", C.c_int32),
        ("activation", C.c_int32), ("message_layers", C.c_int32),
        ("message_mode", C.c_int32), ("message_dim", C.c_int32), ("pair_dim", C.c_int32),
        ("message_groups", C.c_int32), ("vector_channels", C.c_int32),
        ("message_basis_size", C.c_int32), ("equivariant_channels", C.c_int32),
        ("equivariant_l_max", C.c_int32),
        ("message_cutoff", C.c_double), ("norm_eps", C.c_double),
        ("zbl_mode", C.c_int32), ("zbl_rc_inner", C.c_double), ("zbl_rc_outer", C.c_double),
        ("nep_hidden", C.c_int32),
        ("elements", C.POINTER(C.c_char_p)),
    ]


_lib = None


def library():
    """Load the shared library (once); raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
            "g.build()'` or `make -C rune_amd/csrc`. There is no CPU fallback.")
    lib = C.CDLL(str(LIB_PATH))
    vp, i32, i64, f64 = C.c_void_p, C.c_int32, C.c_int64, C.c_double
    sig = {
        "rune_last_error": (C.c_char_p, []),
        "rune_version": (C.c_char_p, []),
        "rune_nlist_create": (C.c_int, [C.POINTER(vp)]),
        "rune_nlist_destroy": (None, [vp]),
        "rune_nlist_build": (C.c_int, [vp, i64, vp, i32, vp, vp, vp, f64, f64, i32, i32, vp,
                                       C.POINTER(i64)]),
        "rune_nlist_update": (C.c_int, [vp, i64, vp, i32, vp, vp, vp, f64, f64, i32, i32, f64,
                                        vp, C.POINTER(i64), C.POINTER(i32)]),
        "rune_nlist_from_padded": (C.c_int, [vp, i64, vp, vp, vp, i32, vp, vp, i32, i32, vp, vp,
                                             C.POINTER(i64)]),
        "rune_nlist_export": (C.c_int, [vp, vp, vp, vp, vp, vp, vp]),
        "rune_nlist_atoms": (i64, [vp]),
        "rune_nlist_records": (i64, [vp]),
        "rune_model_create": (C.c_int, [C.POINTER(ModelConfig), C.POINTER(vp)]),
        "rune_model_destroy": (None, [vp]),
        "rune_model_load": (C.c_int, [C.c_char_p, C.POINTER(vp)]),
        "rune_model_limits": (C.c_int, [vp, C.POINTER(f64), C.POINTER(f64), C.POINTER(i32),
                                        C.POINTER(i32)]),
        "rune_model_element": (C.c_char_p, [vp, i32]),
        "rune_model_compute_gpumd": (C.c_int, [vp, vp, vp, vp, vp, vp, vp]),
        "rune_model_supports_heat_current": (C.c_int, [vp]),
        "rune_model_descriptor_extrema": (C.c_int, [vp, vp, vp, vp, vp, i32, vp]),
        "rune_model_input_dim": (i32, [vp]),
        "rune_model_set_tensor": (C.c_int, [vp, C.c_char_p, vp, i64]),
        "rune_model_finalize": (C.c_int, [vp]),
        "rune_model_compute": (C.c_int, [vp, vp, vp, i32, i32, vp, vp, vp, vp, vp, vp]),
        "rune_model_compute_static": (C.c_int, [vp, vp, vp, i32, i32, vp, vp, vp, vp, vp, vp]),
        "rune_model_static_scratch_bytes": (i64, []),
        "rune_model_workspace_bytes": (i64, [vp]),
        "rune_model_timing": (C.c_int, [vp, i32]),
        "rune_model_timing_read": (C.c_int, [vp, C.POINTER(C.c_double), C.POINTER(i64)]),
        "rune_model_timing_groups": (C.c_int, [vp, C.POINTER(C.c_double), C.POINTER(i64)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc):
    if rc != RUNE_OK:
        msg = library().rune_last_error().decode("utf-8", "replace")
        if rc in (ERR_OVERFLOW, ERR_TYPE, ERR_ARGUMENT):
            raise ValueError(msg)
        raise NativeError(rc, msg)


def require_device(device):
    device = torch.device(device)
    if device.type != "cuda" or not torch.cuda.is_available():
        raise RuntimeError(
            "the rune_amd evaluator runs on an MI355X (HIP) device only; "
            f"got device {device!s} with torch.cuda.is_available()={torch.cuda.is_available()}")
    return device


def compute_device(device=None):
    """HIP device that evaluates for a drop-in object placed on ``device``.

    The reference's calculator and batch builder take a torch ``device``
    (default ``"cpu"``) that decides where the model and its tensors live.
    Here the evaluation always runs on a HIP device: a ``cuda`` device is used
    as given, any other placement (``"cpu"``, ``None``) evaluates on the
    current HIP device and hands results back on the placement device.
    Raises when no HIP device is visible (there is no CPU evaluation path).
    """
    dev = torch.device(device) if device is not None else torch.device("cpu")
    if dev.type == "cuda":
        return require_device(dev)
    if not torch.cuda.is_available():
        raise RuntimeError(
            "the rune_amd evaluator runs on an MI355X (HIP) device only and none is visible "
            f"(placement device {dev!s})")
    return torch.device("cuda", torch.cuda.current_device())


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _stream(device):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class NeighborList:
    """Owner of a ``rune_nlist`` handle (device records, transpose, workspace)."""

    def __init__(self):
        lib = library()
        h = C.c_void_p()
        check(lib.rune_nlist_create(C.byref(h)))
        self._h = h
        self.n_atoms = 0
        self.n_records = 0

    @property
    def handle(self):
        return self._h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and _lib is not None:
            _lib.rune_nlist_destroy(h)
            self._h = None

    def build(self, positions, struct_ptr, cells, pbc, rc_radial, rc_angular, max_radial,
              max_angular):
        """positions: fp64 [N,3] device tensor; struct_ptr, cells, pbc: host sequences."""
        import numpy as np
        pos = positions.contiguous()
        assert pos.dtype == torch.float64 and pos.is_cuda
        sp = np.ascontiguousarray(struct_ptr, dtype=np.int64)
        cl = np.ascontiguousarray(cells, dtype=np.float64).reshape(-1, 9)
        pb = np.ascontiguousarray(pbc, dtype=np.int32).reshape(-1, 3)
        n_rec = C.c_int64()
        check(library().rune_nlist_build(
            self._h, pos.shape[0], _ptr(pos), len(sp) - 1,
            sp.ctypes.data_as(C.c_void_p), cl.ctypes.data_as(C.c_void_p),
            pb.ctypes.data_as(C.c_void_p), float(rc_radial), float(rc_angular),
            int(max_radial), int(max_angular), _stream(pos.device), C.byref(n_rec)))
        self.n_atoms = pos.shape[0]
        self.n_records = n_rec.value
        self.device = pos.device
        self._keep = pos
        return self

    def update(self, positions, struct_ptr, cells, pbc, rc_radial, rc_angular, max_radial,
               max_angular, skin=1.0):
        """As build(), reusing the candidates of the last search while every atom
        stays within skin / 2 of where that search saw it.  Returns True when
        this call searched again."""
        import numpy as np
        pos = positions.contiguous()
        assert pos.dtype == torch.float64 and pos.is_cuda
        sp = np.ascontiguousarray(struct_ptr, dtype=np.int64)
        cl = np.ascontiguousarray(cells, dtype=np.float64).reshape(-1, 9)
        pb = np.ascontiguousarray(pbc, dtype=np.int32).reshape(-1, 3)
        n_rec = C.c_int64()
        searched = C.c_int32()
        check(library().rune_nlist_update(
            self._h, pos.shape[0], _ptr(pos), len(sp) - 1,
            sp.ctypes.data_as(C.c_void_p), cl.ctypes.data_as(C.c_void_p),
            pb.ctypes.data_as(C.c_void_p), float(rc_radial), float(rc_angular),
            int(max_radial), int(max_angular), float(skin), _stream(pos.device),
            C.byref(n_rec), C.byref(searched)))
        self.n_atoms = pos.shape[0]
        self.n_records = n_rec.value
        self.device = pos.device
        self._keep = pos
        return bool(searched.value)

    def from_padded(self, positions, radial_neighbors, radial_offsets, angular_neighbors,
                    angular_offsets, struct_ptr):
        import numpy as np
        pos = positions.contiguous()
        rn = radial_neighbors.to(torch.int64).contiguous()
        an = angular_neighbors.to(torch.int64).contiguous()
        ro = radial_offsets.to(torch.float32).contiguous()
        ao = angular_offsets.to(torch.float32).contiguous()
        sp = np.ascontiguousarray(struct_ptr, dtype=np.int64)
        n_rec = C.c_int64()
        check(library().rune_nlist_from_padded(
            self._h, pos.shape[0], _ptr(pos), _ptr(rn), _ptr(ro), rn.shape[1], _ptr(an),
            _ptr(ao), an.shape[1], len(sp) - 1, sp.ctypes.data_as(C.c_void_p),
            _stream(pos.device), C.byref(n_rec)))
        self.n_atoms = pos.shape[0]
        self.n_records = n_rec.value
        self.device = pos.device
        self._keep = (pos, rn, an, ro, ao)
        return self

    def export(self):
        dev = self.device
        n, e = self.n_atoms, self.n_records
        out = {
            "ptr": torch.empty(n + 1, dtype=torch.int32, device=dev),
            "view": torch.empty((n, 4), dtype=torch.int32, device=dev),
            "nbr": torch.empty(e, dtype=torch.int32, device=dev),
            "shift": torch.empty((e, 3), dtype=torch.int32, device=dev),
            "vec": torch.empty((e, 4), dtype=torch.float32, device=dev),
        }
        check(library().rune_nlist_export(self._h, _ptr(out["ptr"]), _ptr(out["view"]),
                                          _ptr(out["nbr"]), _ptr(out["shift"]), _ptr(out["vec"]),
                                          _stream(dev)))
        return out


def model_config(params, family):
    """``ModelConfig`` from a resolved reference ``model_params`` dict."""
    p = params
    cfg = ModelConfig()
    cfg.family = family
    cfg.n_types = len(p["elements"])
    cfg.n_desc_radial = int(p["n_desc_radial"])
    cfg.k_radial = int(p["k_max_radial"])
    cfg.n_desc_angular = int(p["n_desc_angular"])
    cfg.k_angular = int(p["k_max_angular"])
    cfg.l_max = int(p["l_max"])
    flags = [int(p.get("has_q_222", int(p.get("l_max_4body", 2) > 0))),
             int(p.get("has_q_1111", int(p.get("l_max_5body", 0) > 0))),
             int(p.get("has_q_112", 0)), int(p.get("has_q_123", 0)),
             int(p.get("has_q_233", 0)), int(p.get("has_q_134", 0))]
    for k, v in enumerate(flags):
        cfg.has_q[k] = 1 if v else 0
    cfg.rc_radial = float(p["rcut_radial"])
    cfg.rc_angular = float(p["rcut_angular"])
    if family == FAMILY_MOBIUS:
        cfg.hidden_dim = int(p.get("hidden_dim", 96))
        cfg.ffn_dim = int(p.get("ffn_dim", 2 * cfg.hidden_dim))
        cfg.blocks = int(p.get("blocks", 3))
        cfg.activation = ACT[str(p.get("activation", "silu")).strip().lower()]
        cfg.message_layers = int(p.get("message_layers", 2))
        cfg.message_mode = 1 if p.get("message_mode", "scalar") == "equivariant" else 0
        cfg.message_dim = int(p.get("message_dim", cfg.hidden_dim))
        cfg.pair_dim = int(p.get("pair_dim", 16))
        cfg.message_groups = int(p.get("message_groups", 8))
        cfg.vector_channels = int(p.get("vector_channels", 8))
        cfg.message_basis_size = int(p.get("message_basis_size", p["k_max_radial"]))
        cfg.equivariant_channels = int(p.get("equivariant_channels", 8))
        lq = p.get("equivariant_l_max")
        cfg.equivariant_l_max = int(lq if lq is not None else p["l_max"])
        cfg.message_cutoff = float(p.get("message_cutoff", p["rcut_radial"]))
        cfg.norm_eps = float(p.get("norm_eps", 1e-8))
    else:
        cfg.nep_hidden = int(p["hidden_dims"][0])
    zbl = p.get("zbl")
    if zbl is None:
        cfg.zbl_mode = ZBL_NONE
    else:
        if isinstance(zbl, dict):
            inner, outer = float(zbl["rc_inner"]), float(zbl["rc_outer"])
            flexible = bool(zbl.get("flexible", inner == 0.0 and outer == 0.0))
        else:
            inner, outer = map(float, zbl)
            flexible = inner == 0.0 and outer == 0.0
        cfg.zbl_mode = ZBL_FLEXIBLE if flexible else ZBL_UNIVERSAL
        cfg.zbl_rc_inner, cfg.zbl_rc_outer = inner, outer
    return cfg


class NativeModel:
    """Owner of a ``rune_model`` handle built from params + a state dict."""

    def __init__(self, params, state_dict, family):
        lib = library()
        self.family = family
        cfg = model_config(params, family)
        names = [e.encode() for e in params["elements"]]
        arr = (C.c_char_p * len(names))(*names)
        cfg.elements = C.cast(arr, C.POINTER(C.c_char_p))
        h = C.c_void_p()
        check(lib.rune_model_create(C.byref(cfg), C.byref(h)))
        self._h = h
        try:
            for name, value in state_dict.items():
                if name.endswith("num_batches_tracked"):
                    continue
                t = value.detach().to("cpu", torch.float32).contiguous()
                check(lib.rune_model_set_tensor(h, name.encode(), C.c_void_p(t.data_ptr()),
                                                t.numel()))
            check(lib.rune_model_finalize(h))
        except Exception:
            lib.rune_model_destroy(h)
            self._h = None
            raise

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and _lib is not None:
            _lib.rune_model_destroy(h)
            self._h = None

    def compute(self, nlist, types, n_structures, compute_forces=True, compute_virial=True,
                atom_virial=False, static=False):
        """E + F + virial through ``rune_model_compute``, or with ``static``
        through ``rune_model_compute_static`` (workspace in the library's
        static device scratch; no device allocation by the library)."""
        dev = nlist.device
        n = nlist.n_atoms
        types = types.to(device=dev, dtype=torch.int32).contiguous()
        out = {
            "energies": torch.empty(n, dtype=torch.float32, device=dev),
            "energy": torch.empty(n_structures, dtype=torch.float32, device=dev),
        }
        if compute_forces:
            out["forces"] = torch.empty((n, 3), dtype=torch.float32, device=dev)
        if compute_virial:
            out["virial"] = torch.empty((n_structures, 9), dtype=torch.float32, device=dev)
        if atom_virial:
            out["atom_virial"] = torch.empty((n, 9), dtype=torch.float32, device=dev)
        entry = library().rune_model_compute_static if static else library().rune_model_compute
        check(entry(
            self._h, nlist.handle, _ptr(types), int(compute_forces), int(compute_virial),
            _ptr(out["energies"]), _ptr(out["energy"]), _ptr(out.get("forces")),
            _ptr(out.get("virial")), _ptr(out.get("atom_virial")), _stream(dev)))
        return out

    @classmethod
    def load(cls, path):
        """A model read natively from its text artifact (mobius.txt or nep.txt)."""
        lib = library()
        h = C.c_void_p()
        check(lib.rune_model_load(str(path).encode(), C.byref(h)))
        self = cls.__new__(cls)
        self._h = h
        with open(path, encoding="utf-8") as fh:
            head = fh.readline().split()
        self.family = FAMILY_MOBIUS if head and head[0] == "mobius1" else FAMILY_NEP
        return self

    def limits(self):
        """(rc_radial, rc_angular, max_radial, max_angular); limits are 0 unless
        the model was read from a text artifact."""
        rr, ra, mr, ma = C.c_double(), C.c_double(), C.c_int32(), C.c_int32()
        check(library().rune_model_limits(self._h, C.byref(rr), C.byref(ra), C.byref(mr),
                                          C.byref(ma)))
        return rr.value, ra.value, mr.value, ma.value

    def compute_gpumd(self, nlist, types, potential=None, force=None, virial=None):
        """Adds GPUMD-style fp64 per-atom outputs into the given device arrays
        (potential [N], force [3N] SoA, virial [9N] SoA)."""
        dev = nlist.device
        types = types.to(device=dev, dtype=torch.int32).contiguous()
        for t in (potential, force, virial):
            assert t is None or (t.dtype == torch.float64 and t.is_contiguous())
        check(library().rune_model_compute_gpumd(self._h, nlist.handle, _ptr(types),
                                                 _ptr(potential), _ptr(force), _ptr(virial),
                                                 _stream(dev)))

    def descriptor_extrema(self, nlist, types, q_min=None, q_max=None):
        """Raw-descriptor extrema over the atoms of ``nlist``; pass the previous
        (q_min, q_max) to accumulate over batches.  Returns (q_min, q_max)."""
        dev = nlist.device
        types = types.to(device=dev, dtype=torch.int32).contiguous()
        accumulate = q_min is not None
        if not accumulate:
            n = self.input_dim()
            q_min = torch.empty(n, dtype=torch.float32, device=dev)
            q_max = torch.empty(n, dtype=torch.float32, device=dev)
        check(library().rune_model_descriptor_extrema(self._h, nlist.handle, _ptr(types),
                                                      _ptr(q_min), _ptr(q_max), int(accumulate),
                                                      _stream(dev)))
        return q_min, q_max

    def input_dim(self):
        return int(library().rune_model_input_dim(self._h))

    def supports_heat_current(self):
        return bool(library().rune_model_supports_heat_current(self._h))

    def element(self, t):
        return library().rune_model_element(self._h, int(t)).decode()

    def workspace_bytes(self):
        return int(library().rune_model_workspace_bytes(self._h))

    PHASES = ("descriptor", "dense_fwd", "message_fwd", "readout", "message_bwd", "dense_bwd",
              "reverse", "forces")

    def timing(self, enable=True, phases=True):
        """Kernel-group spans (and, with ``phases``, per-phase events) on or off."""
        check(library().rune_model_timing(self._h, 0 if not enable else (1 if phases else 2)))

    def timing_read(self):
        """Summed milliseconds per phase over the recorded calls, and the call count."""
        ms = (C.c_double * len(self.PHASES))()
        calls = C.c_int64()
        check(library().rune_model_timing_read(self._h, ms, C.byref(calls)))
        return dict(zip(self.PHASES, list(ms))), calls.value

    GROUPS = ("edge_gemm", "edge_kernels")

    def timing_groups(self):
        """Summed milliseconds and launch counts per kernel group since timing was enabled."""
        ms = (C.c_double * len(self.GROUPS))()
        n = (C.c_int64 * len(self.GROUPS))()
        check(library().rune_model_timing_groups(self._h, ms, n))
        return {g: (ms[k], n[k]) for k, g in enumerate(self.GROUPS)}


def version():
    return library().rune_version().decode()


def lib_path():
    return os.fspath(LIB_PATH)
