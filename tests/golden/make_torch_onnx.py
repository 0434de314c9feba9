"""Write tests/golden/torch_export_small.onnx and its parameter file.

The model file is serialised by libtorch's ONNX exporter (the TorchScript
path, whose protobuf writer is compiled into libtorch), i.e. by an
implementation independent of cormorant_amd.scheduler.onnx_io.  The test
decodes it and compares every initializer, attribute and value_info with what
this script records in the .npz file.

The exporter calls the ``onnx`` Python package only to splice in onnx-script
functions (none are used here); that package is absent in this image, so the
splice step is replaced by the identity.

Usage:  python tests/golden/make_torch_onnx.py
"""
import io
import os

import numpy as np
import torch
from torch.onnx._internal.torchscript_exporter import utils as export_utils

HERE = os.path.dirname(os.path.abspath(__file__))


class Small(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.c = torch.nn.Conv2d(3, 8, 3, stride=2, padding=1)
        self.w = torch.nn.Parameter(torch.randn(8, 4))
        self.b = torch.nn.Parameter(torch.randn(4))

    def forward(self, x):
        y = torch.clamp(self.c(x), 0, 6)
        y = torch.nn.functional.max_pool2d(y, 2, 2)
        y = torch.nn.functional.adaptive_avg_pool2d(y, 1)
        y = y.reshape(2, 8)
        return torch.matmul(y, self.w) + self.b


def main():
    torch.manual_seed(42)
    m = Small().eval()
    x = torch.randn(2, 3, 16, 16)
    export_utils.onnx_proto_utils._add_onnxscript_fn = lambda model_bytes, opsets: model_bytes
    f = io.BytesIO()
    torch.onnx.export(m, (x,), f, dynamo=False, opset_version=13, input_names=["X"],
                      output_names=["Y"], do_constant_folding=True)
    with open(os.path.join(HERE, "torch_export_small.onnx"), "wb") as fh:
        fh.write(f.getvalue())
    with torch.no_grad():
        y = m(x)
    np.savez(os.path.join(HERE, "torch_export_small.npz"),
             conv_weight=m.c.weight.detach().numpy(), conv_bias=m.c.bias.detach().numpy(),
             w=m.w.detach().numpy(), b=m.b.detach().numpy(), x=x.numpy(), y=y.numpy())


if __name__ == "__main__":
    main()
