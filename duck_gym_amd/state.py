"""Host-side view of the per-environment HBM state blob.

`StateCodec` decodes the raw bytes exported by `duck_export_state` into
numpy arrays (bodies, joint multipliers, compacted contact lists, colours,
diagnostics) and encodes them back for `duck_import_state`, using the field
offsets the library reports (`duck_state_layout`), so the Python side never
hard-codes the C++ struct layout.  Used by the parity tests to compare the
whole solver state with the CPU oracle and to seed identical states.
"""

from __future__ import annotations

import numpy as np

FIELDS = (
    "B", "J", "CG", "CS", "real", "blob", "header",
    "x", "q", "v", "w", "mass", "inertia", "force", "lambda", "penalty", "lambdaF", "penaltyF",
    "target", "kp", "maxTorque", "torque", "frictionloss", "damping", "diag", "friction",
    "failed", "ngc", "nsc", "colors", "colorCount", "gc", "gcBytes", "sc", "scBytes",
    "gc_id", "gc_local", "gc_anchor", "gc_c0", "gc_lambda", "gc_penalty",
    "sc_id", "sc_local", "sc_localB", "sc_t1", "sc_t2", "sc_n", "sc_c0", "sc_friction",
    "sc_lambda", "sc_penalty",
)
# (field, components) of body-indexed [k][B] and joint-indexed [k][J] arrays.
BODY = (("x", 3), ("q", 4), ("v", 3), ("w", 3), ("mass", 1), ("inertia", 3))
JOINT = (("lambda", 7), ("penalty", 7), ("lambdaF", 1), ("penaltyF", 1), ("target", 1),
         ("kp", 1), ("maxTorque", 1), ("torque", 1), ("frictionloss", 1), ("damping", 1))
GROUND = (("local", 3), ("anchor", 2), ("c0", 1), ("lambda", 3), ("penalty", 3))
SELF = (("local", 3), ("localB", 3), ("t1", 3), ("t2", 3), ("n", 3), ("c0", 1),
        ("friction", 1), ("lambda", 3), ("penalty", 3))


def ground_id(shape, body, feature, stick=False):
    v = shape | (body << 6) | (feature << 12) | (0x80000000 if stick else 0)
    return np.int32(np.uint32(v).view(np.int32))


def self_id(body, other, shape, other_shape, stick=False):
    v = body | (other << 6) | (shape << 12) | (other_shape << 18) | (0x80000000 if stick else 0)
    return np.int32(np.uint32(v).view(np.int32))


class StateCodec:
    def __init__(self, layout, bodies, joints):
        self.L = dict(zip(FIELDS, (int(v) for v in layout)))
        self.nb, self.nj = bodies, joints
        self.dtype = np.float64 if self.L["real"] == 8 else np.float32
        self.rb = self.L["real"]

    def _reals(self, raw, off, n):
        return np.frombuffer(raw[off: off + n * self.rb].tobytes(), dtype=self.dtype).copy()

    def _ints(self, raw, off, n):
        return np.frombuffer(raw[off: off + 4 * n].tobytes(), dtype=np.int32).copy()

    def decode(self, raw):
        """raw: uint8 array of one blob -> dict of numpy arrays."""
        L, B, J = self.L, self.L["B"], self.L["J"]
        raw = np.asarray(raw, dtype=np.uint8)
        out = {}
        for name, k in BODY:
            a = self._reals(raw, L[name], k * B).reshape(k, B)[:, : self.nb]
            out[name] = a.T.copy() if k > 1 else a[0].copy()
        for name, k in JOINT:
            a = self._reals(raw, L[name], k * J).reshape(k, J)[:, : self.nj]
            out[name] = a.T.copy() if k > 1 else a[0].copy()
        out["force"] = self._reals(raw, L["force"], 3)
        out["diag"] = self._reals(raw, L["diag"], 8)
        out["friction"] = self._reals(raw, L["friction"], 1)[0]
        out["failed"], out["ngc"], out["nsc"], out["colorCount"] = (
            int(self._ints(raw, L[f], 1)[0]) for f in ("failed", "ngc", "nsc", "colorCount"))
        out["colors"] = self._ints(raw, L["colors"], B)[: self.nb]
        gcs = []
        for i in range(out["ngc"]):
            base = L["gc"] + i * L["gcBytes"]
            c = {"id": int(self._ints(raw, base + L["gc_id"], 1)[0])}
            for name, k in GROUND:
                c[name] = self._reals(raw, base + L["gc_" + name], k)
            c["shape"], c["body"] = c["id"] & 63, (c["id"] >> 6) & 63
            c["feature"], c["stick"] = (c["id"] >> 12) & 0x7FFFF, c["id"] < 0
            gcs.append(c)
        out["gc"] = gcs
        scs = []
        for i in range(out["nsc"]):
            base = L["sc"] + i * L["scBytes"]
            c = {"id": int(self._ints(raw, base + L["sc_id"], 1)[0])}
            for name, k in SELF:
                c[name] = self._reals(raw, base + L["sc_" + name], k)
            c["body"], c["other"] = c["id"] & 63, (c["id"] >> 6) & 63
            c["shape"], c["otherShape"], c["stick"] = (c["id"] >> 12) & 63, (c["id"] >> 18) & 63, c["id"] < 0
            scs.append(c)
        out["sc"] = scs
        return out

    def _put(self, raw, off, values, dtype):
        b = np.ascontiguousarray(values, dtype=dtype).tobytes()
        raw[off: off + len(b)] = np.frombuffer(b, dtype=np.uint8)

    def encode(self, raw, s):
        """Write the fields of decoded dict `s` into the uint8 blob `raw` (in place)."""
        L, B, J = self.L, self.L["B"], self.L["J"]
        for name, k in BODY:
            a = np.zeros((k, B))
            v = np.asarray(s[name], dtype=np.float64)
            a[:, : self.nb] = v.T if k > 1 else v[None]
            self._put(raw, L[name], a.ravel(), self.dtype)
        for name, k in JOINT:
            a = np.zeros((k, J))
            v = np.asarray(s[name], dtype=np.float64)
            a[:, : self.nj] = v.T if k > 1 else v[None]
            self._put(raw, L[name], a.ravel(), self.dtype)
        self._put(raw, L["force"], s["force"], self.dtype)
        self._put(raw, L["diag"], s["diag"], self.dtype)
        self._put(raw, L["friction"], [s["friction"]], self.dtype)
        for f in ("failed", "ngc", "nsc", "colorCount"):
            self._put(raw, L[f], [s[f]], np.int32)
        colors = np.zeros(B, dtype=np.int32)
        colors[: self.nb] = s["colors"]
        self._put(raw, L["colors"], colors, np.int32)
        for i, c in enumerate(s["gc"]):
            base = L["gc"] + i * L["gcBytes"]
            self._put(raw, base + L["gc_id"], [c["id"]], np.int32)
            for name, k in GROUND:
                self._put(raw, base + L["gc_" + name], c[name], self.dtype)
        for i, c in enumerate(s["sc"]):
            base = L["sc"] + i * L["scBytes"]
            self._put(raw, base + L["sc_id"], [c["id"]], np.int32)
            for name, k in SELF:
                self._put(raw, base + L["sc_" + name], c[name], self.dtype)
        return raw
