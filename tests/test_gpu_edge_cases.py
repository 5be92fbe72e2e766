"""GPU parity at the edges of the input space (tests/edge_instances.py): the smallest instance, empty tensors,
labels held by one tensor, open labels, every register width and the first runtime width, both sweep orders,
float node costs, and chain counts that leave workgroups partly filled -- the HIP path through the C ABI
against the oracle, bit for bit (records, counts, energies)."""
import pytest

import edge_instances as E
from test_gpu_parity import Case, compare

pytestmark = pytest.mark.gpu

CASES = [(n, o, c, 0) for n in E.NAMES for o, c in (("par", 65), ("preorder", 5))]
CASES += [("mixed40", "par", 1, 1), ("deg3_129", "par", 3, 2), ("deg3_513", "preorder", 1, 0)]


@pytest.mark.parametrize("name,order,nchains,mode", CASES, ids=[f"{n}-{o}-{c}-m{k}" for n, o, c, k in CASES])
def test_edge_instance_matches_oracle(name, order, nchains, mode):
    case = Case(name, order, mode, init="random", nchains=nchains, data=E.instance(name))
    compare(case, case.run_gpu(), case.run_oracle())
