"""GPU parity at the edges of the input space (tests/edge_instances.py): the smallest instance, empty tensors,
labels held by one tensor, open labels, every register width and the first runtime width, the largest chain
whose par scan keeps a list of unvisited nodes (512 internal nodes) and the next one, both sweep orders,
float node costs, and chain counts that leave workgroups partly filled -- the HIP path through the C ABI
against the oracle, bit for bit (records, counts, energies)."""
import numpy as np
import pytest

import edge_instances as E
from treesa_gpu_amd import capi
from test_gpu_parity import Case, compare

pytestmark = pytest.mark.gpu

CASES = [(n, o, c, 0) for n in E.NAMES for o, c in (("par", 65), ("preorder", 5))]
CASES += [("mixed40", "par", 1, 1), ("deg3_129", "par", 3, 2), ("deg3_513", "preorder", 1, 0)]
CASES += [(n, o, 3, 0) for n in E.WIDE for o in ("par", "preorder")]


@pytest.mark.parametrize("name,order,nchains,mode", CASES, ids=[f"{n}-{o}-{c}-m{k}" for n, o, c, k in CASES])
def test_edge_instance_matches_oracle(name, order, nchains, mode):
    case = Case(name, order, mode, init="random", nchains=nchains, data=E.instance(name))
    gpu = case.run_gpu()
    if name == "wide_16384" and order == "par":
        assert "wide" in gpu[3], gpu[3]  # the widest chain the wide kernel takes
    if name == "wide_16385":
        assert "wide" not in gpu[3], gpu[3]  # past it: the one-wave kernel with runtime width
    if name.startswith("sparse_"):
        assert gpu[3].startswith("lds"), gpu[3]  # the chain in LDS: the par scan's list or its full form
    compare(case, gpu, case.run_oracle())


def test_largest_node_ids_do_not_fit_the_node_arrays():
    """m = 32768 tensors (node ids up to 65534, the 16-bit limit) is accepted by the layout; the par sweep's
    per-node arrays then exceed LDS, which creation reports as a fit error before any kernel runs."""
    m, nlab = 32768, 3
    lay = capi.layout(m, nlab)
    leaf = np.zeros((m, lay.W), np.uint64)
    leaf[:, 0] = np.uint64(1)
    with pytest.raises(capi.TsaError, match="fit"):
        capi.Context(lay, leaf, 1, capi.make_config(), 4)
