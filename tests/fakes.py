"""The stand-ins of fairseq / fairscale / apex objects the tests drive the drop-in surfaces through (they live in the
package, faster_yoco_amd.standins, where bench.py also uses them)."""
from faster_yoco_amd.standins import (FakeCEReduce, FakeFairseqOptimizer, FakeFP16Optimizer,  # noqa: F401
                                      FakeFusedAdamV2, FakeMixin, FakeOSS)
