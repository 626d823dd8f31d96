"""ctypes wrapper of the C oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module.  It binds oracle/_build/liboracle.so (built by oracle/Makefile)
and feeds it the tensors of a `.so3lr` model read by oracle/model_io.py.
"""
import ctypes
import os
import subprocess

import numpy as np

from . import model_io

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

HW, MAXL, MAXS = 32, 8, 8
NORM_LAYER, NORM_RMS, NORM_NONE = 0, 1, 2
REP_ZBL, REP_NLH = 0, 1

GLOBAL_KEYS = [
    "model.inv_feature_embedding.embedding.weight",
    "model.radial_embedding.radial_basis_fn.b",
    "model.atomic_energy_output_block.layers.0.weight",
    "model.atomic_energy_output_block.layers.0.bias",
    "model.atomic_energy_output_block.final_layer.weight",
    "model.atomic_energy_output_block.final_layer.bias",
    "model.atomic_energy_output_block.energy_scales.weight",
    "model.atomic_energy_output_block.energy_shifts",
    "model.partial_charges_output_block.atomic_embedding.weight",
    "model.partial_charges_output_block.transform_inv_features.0.weight",
    "model.partial_charges_output_block.transform_inv_features.0.bias",
    "model.partial_charges_output_block.transform_inv_features.2.weight",
    "model.partial_charges_output_block.transform_inv_features.2.bias",
    "model.hirshfeld_output_block.q_embedding.weight",
    "model.hirshfeld_output_block.transform_features.0.weight",
    "model.hirshfeld_output_block.transform_features.0.bias",
    "model.hirshfeld_output_block.transform_features.2.weight",
    "model.hirshfeld_output_block.transform_features.2.bias",
    "model.hirshfeld_output_block.v_shift_embedding.weight",
    "model.charge_embedding.Wq.weight",
    "model.charge_embedding.Wk",
    "model.charge_embedding.Wv",
    "model.charge_embedding.mlp.1.weight",
    "model.charge_embedding.mlp.3.weight",
    "model.spin_embedding.Wq.weight",
    "model.spin_embedding.Wk",
    "model.spin_embedding.Wv",
    "model.spin_embedding.mlp.1.weight",
    "model.spin_embedding.mlp.3.weight",
    "physical.reference_alphas",
    "physical.reference_c6",
    # the optional C6 ratio head (absent from v1 models)
    "model.c6_ratios_output_block.q_embedding.weight",
    "model.c6_ratios_output_block.transform_features.0.weight",
    "model.c6_ratios_output_block.transform_features.0.bias",
    "model.c6_ratios_output_block.transform_features.2.weight",
    "model.c6_ratios_output_block.transform_features.2.bias",
    "model.c6_ratios_output_block.v_shift_embedding.weight",
]

_FILTER = ["mlp_rbf.0.weight", "mlp_rbf.0.bias", "mlp_rbf.mlp_rbf_layer_1.0.weight",
           "mlp_rbf.mlp_rbf_layer_1.0.bias", "mlp_ev.0.weight", "mlp_ev.0.bias",
           "mlp_ev.mlp_ev_layer_1.0.weight", "mlp_ev.mlp_ev_layer_1.0.bias"]


def block_keys(b):
    p = "model.euclidean_transformers.%d." % b
    a = p + "euclidean_attention_block."
    keys = [a + "W_q_inv", a + "W_k_inv", a + "W_v_inv", a + "W_q_ev", a + "W_k_ev"]
    # The filter nets the reference evaluates live at the transformer level
    # (kokkos_integrated_block0.cpp:507-512).
    keys += [p + "filter_net_inv." + s for s in _FILTER]
    keys += [p + "filter_net_ev." + s for s in _FILTER]
    keys += [a + "so3_conv_invariants.cg_rep", p + "interaction_block.so3_conv_invariants.cg_rep"]
    keys += [p + "layer_norm_inv_1.weight", p + "layer_norm_inv_1.bias",
             p + "mlp_1.1.weight", p + "mlp_1.1.bias", p + "mlp_1.3.weight", p + "mlp_1.3.bias",
             p + "interaction_block.linear_layer.weight", p + "interaction_block.linear_layer.bias",
             p + "layer_norm_inv_2.weight", p + "layer_norm_inv_2.bias"]
    return keys


SCALAR_KEYS = [
    # (architecture key) in orc scalar order; gamma comes from a tensor
    None, "short_range_cutoff_angstrom", "avg_num_neighbors", "embedding_scale",
    "layer_norm_epsilon",
    "zbl_ke", "zbl_switch_off_angstrom", "zbl_p", "zbl_d",
    "zbl_a1", "zbl_a2", "zbl_a3", "zbl_a4", "zbl_c1", "zbl_c2", "zbl_c3", "zbl_c4",
    "lr_electrostatic_ke", "lr_electrostatic_sigma", "long_range_cutoff_angstrom",
    "lr_electrostatic_cuton_angstrom", "lr_fine_structure", "lr_bohr_angstrom",
    "lr_hartree_ev", "lr_dispersion_scale", "lr_dispersion_cuton_angstrom", "lr_pair_scale",
]

NTENSOR = len(GLOBAL_KEYS) + MAXL * len(block_keys(0))


class _Model(ctypes.Structure):
    _fields_ = [("t", ctypes.c_void_p * NTENSOR),
                ("rbf_k", ctypes.c_void_p),
                ("rbf_krev", ctypes.c_void_p),
                ("n_alpha_ref", ctypes.c_int64),
                ("s", ctypes.c_double * len(SCALAR_KEYS)),
                ("n_blocks", ctypes.c_int64),
                ("norm1", ctypes.c_int64),
                ("norm2", ctypes.c_int64),
                ("qk_norm", ctypes.c_int64),
                ("repulsion", ctypes.c_int64),
                ("nlh_cap", ctypes.c_int64),
                ("nlh_a", ctypes.c_void_p),
                ("nlh_b", ctypes.c_void_p),
                ("resid", ctypes.c_void_p),
                ("x0l", ctypes.c_void_p),
                ("F", ctypes.c_int64),
                ("R", ctypes.c_int64),
                ("n_slots", ctypes.c_int64),
                ("degrees", ctypes.c_int64 * MAXS),
                ("head_hidden", ctypes.c_int64)]


class _Out(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in
                ("e_learned", "e_zbl", "e_lr", "charges", "hirshfeld", "forces", "virial",
                 "image_energy", "vatom", "c6_ratios")] + [
                ("e_elec_total", ctypes.c_double), ("e_disp_total", ctypes.c_double),
                ("e_total", ctypes.c_double)]


def build():
    """Compile the oracle (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.orc_evaluate.restype = ctypes.c_int
        _lib.orc_charge_spin_table.restype = ctypes.c_int
        _lib.orc_charge_multiplicity_problem.restype = ctypes.c_int
        _lib.orc_num_threads.restype = ctypes.c_int
        _lib.orc_rms_rows.restype = None
    return _lib


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


class Oracle:
    """Holds one model's tensors for the C oracle."""

    def __init__(self, model_path):
        self.model = model_io.load(model_path)
        m = self.model
        arch = m.arch
        self._keep = []
        st = _Model()
        nb = int(arch["interaction_blocks"])
        if not 1 <= nb <= MAXL:
            raise ValueError("interaction_blocks outside 1..%d" % MAXL)
        keys = list(GLOBAL_KEYS)
        for b in range(MAXL):
            keys += block_keys(b) if b < nb else [None] * len(block_keys(0))
        assert len(keys) == NTENSOR
        for i, k in enumerate(keys):
            if k is None or k not in m.tensors:
                st.t[i] = None  # absent: the C6 head of a v1 model, parameter-free norms
                continue
            st.t[i] = self._hold(m[k], np.float64)
        k = np.ascontiguousarray(m["model.radial_embedding.radial_basis_fn.k"], dtype=np.int64)
        kr = np.ascontiguousarray(m["model.radial_embedding.radial_basis_fn.k_rev"], dtype=np.int64)
        self._keep += [k, kr]
        st.rbf_k = k.ctypes.data
        st.rbf_krev = kr.ctypes.data
        st.n_alpha_ref = m["physical.reference_alphas"].shape[0]
        for i, key in enumerate(SCALAR_KEYS):
            if key is None:
                st.s[i] = float(m["model.radial_embedding.radial_basis_fn.gamma"])
            elif key == "avg_num_neighbors":
                st.s[i] = attention_norm(arch)
            elif key in arch:
                st.s[i] = float(arch[key])
            elif key.startswith("zbl_") and arch.get("repulsion_type") == "nlh":
                st.s[i] = 0.0  # learned-ZBL parameters: not part of an NLH model
            else:
                raise KeyError(key)
        # architecture options (so3lr_architecture.cpp:356-392)
        st.n_blocks = nb
        enabled = NORM_RMS if arch.get("use_rms_norm", False) else NORM_LAYER
        st.norm1 = enabled if arch.get("layer_normalization_1", True) else NORM_NONE
        st.norm2 = enabled if arch.get("layer_normalization_2", True) else NORM_NONE
        st.qk_norm = 1 if arch.get("qk_norm", False) else 0
        if arch.get("repulsion_type", "zbl_learned") == "nlh":
            st.repulsion = REP_NLH
            a = m["physical.nlh_a"]
            st.nlh_cap = a.shape[0]
            st.nlh_a = self._hold(a, np.float64)
            st.nlh_b = self._hold(m["physical.nlh_b"], np.float64)
        if arch.get("use_residual_scalars", False):
            st.resid = self._hold(m["model.resid_lambdas"], np.float64)
            st.x0l = self._hold(m["model.x0_lambdas"], np.float64)
        self.has_c6 = "model.c6_ratios_output_block.transform_features.0.weight" in m.tensors
        # widths (so3lr_architecture.cpp:197-212, 246-293, 444-446)
        self.F = int(arch["invariant_features"])
        st.F = self.F
        st.R = int(arch["radial_basis_features"])
        rep = [int(v) for v in m["model.euclidean_transformers.0.euclidean_attention_block.degree_repeats"]]
        if len(rep) > MAXS:
            raise ValueError("more than %d degree slots" % MAXS)
        st.n_slots = len(rep)
        for s, v in enumerate(rep):
            st.degrees[s] = (v - 1) // 2
        st.head_hidden = m["model.atomic_energy_output_block.layers.0.weight"].shape[0]
        self._st = st

    def _hold(self, a, dtype):
        arr = np.ascontiguousarray(a, dtype=dtype)
        self._keep.append(arr)
        return arr.ctypes.data

    def charge_spin_table(self, counts, charge, multiplicity):
        counts = np.ascontiguousarray(counts, dtype=np.int64)
        table = np.zeros((118, self.F))
        rc = lib().orc_charge_spin_table(ctypes.byref(self._st), _ptr(counts),
                                         ctypes.c_double(charge),
                                         ctypes.c_double(multiplicity - 1.0), _ptr(table))
        if rc != 0:
            raise RuntimeError("charge/spin table failed")
        return table

    @staticmethod
    def charge_multiplicity_problem(counts, charge, multiplicity):
        counts = np.ascontiguousarray(counts, dtype=np.int64)
        return lib().orc_charge_multiplicity_problem(_ptr(counts), ctypes.c_double(charge),
                                                     ctypes.c_double(multiplicity))

    def evaluate(self, z, sr, lr, charge=0.0, multiplicity=1.0, image=None,
                 image_charge=None, image_multiplicity=None):
        """E + F + virial.

        sr = (senders, receivers, vectors) directed edges, v = x_r - x_s;
        lr = (pi, pj, vectors) unique half pairs, d = x_pj - x_pi.
        For packed images pass image ids and per-image charge/multiplicity.
        """
        z = np.ascontiguousarray(z, dtype=np.int64)
        n = len(z)
        if image is None:
            counts = np.bincount(z, minlength=119).astype(np.int64)
            table = self.charge_spin_table(counts, charge, multiplicity)
            offset = np.ascontiguousarray(table[z - 1])
            n_images = 1
            img = None
            img_q = np.array([float(charge)])
        else:
            img = np.ascontiguousarray(image, dtype=np.int64)
            n_images = int(img.max()) + 1
            img_q = np.ascontiguousarray(image_charge, dtype=np.float64)
            offset = np.zeros((n, self.F))
            for k in range(n_images):
                sel = img == k
                counts = np.bincount(z[sel], minlength=119).astype(np.int64)
                table = self.charge_spin_table(counts, img_q[k], image_multiplicity[k])
                offset[sel] = table[z[sel] - 1]
        snd, rcv, vec = (np.ascontiguousarray(a) for a in sr)
        snd = snd.astype(np.int64); rcv = rcv.astype(np.int64); vec = vec.astype(np.float64)
        pi, pj, pvec = (np.ascontiguousarray(a) for a in lr)
        pi = pi.astype(np.int64); pj = pj.astype(np.int64); pvec = pvec.astype(np.float64)
        outs = {k: np.zeros(n) for k in ("e_learned", "e_zbl", "e_lr", "charges", "hirshfeld")}
        outs["forces"] = np.zeros((n, 3))
        outs["virial"] = np.zeros(6)
        outs["vatom"] = np.zeros((n, 6))
        outs["image_energy"] = np.zeros(n_images)
        if self.has_c6:
            outs["c6_ratios"] = np.zeros(n)
        o = _Out()
        for k, v in outs.items():
            setattr(o, k, v.ctypes.data)
        rc = lib().orc_evaluate(
            ctypes.byref(self._st), ctypes.c_int64(n), _ptr(z), _ptr(offset),
            ctypes.c_int64(n_images), _ptr(img), _ptr(img_q),
            ctypes.c_int64(len(snd)), _ptr(snd), _ptr(rcv), _ptr(vec),
            ctypes.c_int64(len(pi)), _ptr(pi), _ptr(pj), _ptr(pvec), ctypes.byref(o))
        if rc != 0:
            raise RuntimeError("orc_evaluate failed with code %d" % rc)
        outs["e_elec_total"] = o.e_elec_total
        outs["e_disp_total"] = o.e_disp_total
        outs["energy"] = o.e_total
        outs["eatom"] = outs["e_learned"] + outs["e_zbl"] + outs["e_lr"]
        return outs


def attention_norm(arch):
    """The divisor of the attention logits (so3lr_architecture.cpp:340-355):
    1, sqrt(attention_head_width) or avg_num_neighbors, by
    message_normalization (avg_num_neighbors when the key is absent)."""
    kind = arch.get("message_normalization", "avg_num_neighbors")
    if kind == "identity":
        return 1.0
    if kind == "sqrt_num_features":
        return float(np.sqrt(float(arch["attention_head_width"])))
    if kind == "avg_num_neighbors":
        return float(arch["avg_num_neighbors"])
    raise ValueError("unknown message_normalization %r" % kind)


def rms_rows(x, eps):
    """orc_rms_rows over the rows of x (2-D): (y, 1 / rms per row)."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.zeros_like(x)
    r = np.zeros(x.shape[0])
    lib().orc_rms_rows(ctypes.c_int64(x.shape[0]), ctypes.c_int64(x.shape[1]), _ptr(x), ctypes.c_double(eps),
                       _ptr(y), _ptr(r))
    return y, r


def spherical_harmonics(u):
    """Y_{1..4}(u) for unit vectors u[n,3] (24 values each), via the C oracle."""
    u = np.ascontiguousarray(u, dtype=np.float64).reshape(-1, 3)
    out = np.zeros((len(u), 24))
    f = lib().orc_spherical_harmonics
    f.restype = None
    buf = np.zeros(24)
    for k in range(len(u)):
        f(ctypes.c_double(u[k, 0]), ctypes.c_double(u[k, 1]), ctypes.c_double(u[k, 2]),
          buf.ctypes.data_as(ctypes.c_void_p))
        out[k] = buf
    return out
