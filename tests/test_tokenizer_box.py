"""The tokenizer suite (the reference's 39 tests of data/tokenizer.rs:517-921
plus the library-vs-restatement parity) run again on the GPU box, against the
librtgpu.so that travels there. The tokenizer is host code: these tests need
no GPU, but the -m gpu run is the one that executes on the box."""
import pytest

from tests.test_tokenizer import *  # noqa: F401,F403 - re-collected here under the gpu mark

pytestmark = pytest.mark.gpu
