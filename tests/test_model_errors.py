"""The boundary's model-file errors, through the product's own loader
(duck_gym_amd/csrc/duck_model.cpp via duck_model_info, no device needed):
every rejection of Solver::load (src/solver.cpp:67-174, a std::runtime_error
-> RuntimeError) and of the flattening and backend checks (model.hpp:26-91,
std::invalid_argument -> ValueError; extension.cu:225-236 and 424,
TORCH_CHECK -> RuntimeError), each with the reference's message.

The unreachable check is the bipartite-graph test (model.hpp:84-87): every
hinge joins a body to its single, earlier parent, so depth-parity colours
always differ across a hinge of two dynamic bodies.
"""

import pytest

from duck_gym_amd.native import check_model
from model_text import chain

NB = 4  # world + 3 links; lines: header, gravity, bodies 2..5, hinges 6..7, shapes 8..10


def _set(index, text):
    def edit(lines):
        lines[index] = text
    return edit


def _field(index, position, value):
    def edit(lines):
        parts = lines[index].split()
        parts[position] = str(value)
        lines[index] = " ".join(parts)
    return edit


BODY1, HINGE0, SHAPE0 = 3, 2 + NB, 2 + NB + (NB - 2)
RUNTIME = [
    ("header magic", chain(header="DUCK_MODLE 2 4 2 3"), "Invalid model header"),
    ("header version", chain(header="DUCK_MODEL 3 4 2 3"), "Invalid model header"),
    ("no bodies", chain(header="DUCK_MODEL 2 0 2 3"), "Invalid model header"),
    ("negative joint count", chain(header="DUCK_MODEL 2 4 -1 3"), "Invalid model header"),
    ("negative mass", chain(edit=_field(BODY1, 1, -0.1)), "Invalid mass/inertia"),
    ("zero inertia", chain(edit=_field(BODY1, 3, 0)), "Invalid mass/inertia"),
    ("zero quaternion", chain(edit=lambda l: [_field(BODY1, k, 0)(l) for k in (8, 9, 10, 11)]),
     "Zero quaternion"),
    ("hinge to itself", chain(edit=_field(HINGE0, 2, 1)), "Invalid joint"),
    ("hinge body out of range", chain(edit=_field(HINGE0, 2, 9)), "Invalid joint"),
    ("negative damping", chain(edit=_field(HINGE0, 24, -1)), "Invalid joint"),
    ("negative armature", chain(edit=_field(HINGE0, 25, -1)), "Invalid joint"),
    ("negative friction loss", chain(edit=_field(HINGE0, 26, -1)), "Invalid joint"),
    ("zero hinge axis", chain(edit=lambda l: [_field(HINGE0, k, 0)(l) for k in (9, 10, 11)]),
     "Zero direction"),
    ("shape kind", chain(edit=_field(SHAPE0, 1, 4)), "Invalid collision shape"),
    ("shape body", chain(edit=_field(SHAPE0, 0, 7)), "Invalid collision shape"),
    ("shape friction", chain(edit=_field(SHAPE0, 12, -0.5)), "Invalid collision shape"),
    ("hull of three points", chain(edit=_set(SHAPE0, "1 3 0 0 0 1 0 0 0 0 0 0 0.8 3 "
                                                     "0 0 0 0.01 0 0 0 0.01 0 1")),
     "Convex mesh needs at least four vertices"),
    ("pair count", chain(edit=lambda l: l.__setitem__(-1, "33")), "Invalid body collision pair count"),
    ("pair on one body", chain(bodies=3, shapes_per_body=2, pairs=[(0, 1, 0.5)]),
     "Invalid body collision pair"),
    ("pair order", chain(pairs=[(1, 0, 0.5)]), "Invalid body collision pair"),
    ("pair friction", chain(pairs=[(0, 2, -1)]), "Invalid body collision pair"),
    ("duplicate pair", chain(pairs=[(0, 2, 0.5), (0, 2, 0.6)]), "Duplicate body collision pair"),
    ("truncated", chain(pairs=[(0, 2, 0.5)])[:-4], "Truncated model"),
    ("trailing data", chain(extra="42\n"), "Unexpected model data"),
]

VALUE = [
    ("33 bodies", chain(bodies=33), "capacity exceeded (32 bodies/joints/shapes)"),
    ("33 pairs", None, "Invalid body collision pair count"),  # the parser's limit comes first
    ("world only", "DUCK_MODEL 1 1 0 0\n0 0 -9.81 1\nworld 0 0 0 0 0 0 0 1 0 0 0 0 0 0 0 0 0\n",
     "at least one body"),
    # five bodies: hinges on lines 7-9; the third becomes 1 -> 3 (body 3's second parent)
    ("two parents", chain(bodies=5, edit=lambda l: (_field(9, 1, 1)(l), _field(9, 2, 3)(l))),
     "at most one parent hinge"),
    ("child before parent", chain(edit=lambda l: (_field(HINGE0, 1, 2)(l), _field(HINGE0, 2, 1)(l))),
     "topological body ordering"),
    ("joint list order", chain(edit=lambda l: l.__setitem__(slice(HINGE0, HINGE0 + 2),
                                                            [l[HINGE0 + 1], l[HINGE0]])),
     "parent-before-child ordering"),
]


@pytest.mark.parametrize("name,text,message", RUNTIME, ids=[c[0] for c in RUNTIME])
def test_malformed_files_raise_runtime_error(tmp_path, name, text, message):
    path = tmp_path / "m.duck"
    path.write_text(text)
    with pytest.raises(RuntimeError, match=message):
        check_model(path)


@pytest.mark.parametrize("name,text,message", [c for c in VALUE if c[1] is not None],
                         ids=[c[0] for c in VALUE if c[1] is not None])
def test_model_contract_violations_raise_value_error(tmp_path, name, text, message):
    path = tmp_path / "m.duck"
    path.write_text(text)
    with pytest.raises(ValueError, match=message.replace("(", r"\(").replace(")", r"\)")):
        check_model(path)


def test_unreadable_file(tmp_path):
    with pytest.raises(RuntimeError, match="Cannot read model"):
        check_model(tmp_path / "absent.duck")
    (tmp_path / "dir.duck").mkdir()
    with pytest.raises(RuntimeError):
        check_model(tmp_path / "dir.duck")


def test_valid_models_report_counts(tmp_path, models):
    path = tmp_path / "m.duck"
    path.write_text(chain(bodies=6, shapes_per_body=2, pairs=[(0, 3, 0.5), (1, 6, 0.4)]))
    assert check_model(path) == dict(bodies=6, joints=4, shapes=10, pairs=2,
                                     ground_capacity=40, self_capacity=2)
    # v1 file: no ground flags (all shapes touch the ground), no pairs
    path.write_text(chain(version=1))
    assert check_model(path)["ground_capacity"] == 12
    # the largest generic model: 32 bodies, 30 hinges, 32 shapes, 32 pairs
    path.write_text(chain(bodies=32, shapes_per_body=1,
                          pairs=[(a, a + 2, 0.5) for a in range(29)] + [(0, 5, .5), (0, 6, .5), (0, 7, .5)]))
    info = check_model(path)
    assert info["ground_capacity"] + info["self_capacity"] == 4 * 31 + 32 <= 160
    info = check_model(models["selfc"], specialized=True, shared_memory=True)
    assert (info["bodies"], info["joints"]) == (16, 14)


def test_specialized_backend_checks(tmp_path, models):
    """MicroDuckState<16, 14, 64>: capacities are ValueErrors (convert),
    the exact layout RuntimeErrors (the Batch constructor)."""
    path = tmp_path / "m.duck"
    path.write_text(chain(bodies=17))
    with pytest.raises(ValueError, match="body/joint capacity"):
        check_model(path, specialized=True)
    path.write_text(chain(bodies=16, shapes_per_body=1, edit=None).replace(
        "DUCK_MODEL 2 16 14 15", "DUCK_MODEL 2 16 14 17") .rstrip("\n").rsplit("\n", 1)[0]
        + "\n1 1 0 0 0 1 0 0 0 0.03 0.02 0.02 0.8 0 1\n2 1 0 0 0 1 0 0 0 0.03 0.02 0.02 0.8 0 1\n0\n")
    assert check_model(path)["ground_capacity"] == 68
    with pytest.raises(ValueError, match="contact capacity"):
        check_model(path, specialized=True)
    path.write_text(chain(bodies=10))
    with pytest.raises(RuntimeError, match="requires 16 bodies and 14 hinges"):
        check_model(path, specialized=True)
    path.write_text(chain(bodies=16))
    with pytest.raises(RuntimeError, match="Unsupported MicroDuck joint layout"):
        check_model(path, specialized=True)
    with pytest.raises(RuntimeError, match="Shared memory requires the compact MicroDuck backend"):
        check_model(models["standing"], shared_memory=True)


REF_DIR = __import__("pathlib").Path(__file__).resolve().parents[1] / "oracle" / "_ref"


@pytest.mark.skipif(not any(REF_DIR.glob("_duck_reference*.so")),
                    reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("case", RUNTIME + [c for c in VALUE if c[1] is not None],
                         ids=[c[0] for c in RUNTIME + [c for c in VALUE if c[1] is not None]])
def test_reference_build_raises_the_same(tmp_path, case):
    """The reference's own CPU batch (src/cuda/cpu_bindings.cpp, compiled in
    place: Solver::load then convert<State>) rejects each file with the same
    exception type and message."""
    import sys

    sys.path.insert(0, str(REF_DIR))
    import _duck_reference

    name, text, message = case
    path = tmp_path / "m.duck"
    path.write_text(text)
    expected = ValueError if case in VALUE else RuntimeError
    with pytest.raises(expected) as caught:
        _duck_reference.CpuBatch32(str(path), 1, 0.005, 10, 1)
    assert message in str(caught.value), (name, str(caught.value))
