"""tiga (MI355X provider): Tiga's CSR message-passing API over gfx950 HIP kernels.

Public names follow the reference package (python/tiga/__init__.py:45-66):
``tiga.MessagePassing``, ``tiga.Graph``, ``tiga.sum``, ``tiga.online_softmax``.
"""

from . import interop, nn, reducer
from .graph import Graph, GraphSchema
from .kernel import CompiledVariant, Kernel
from .message_passing import MessagePassing, config
from .reducer import (
    OnlineSoftmaxItem,
    OnlineSoftmaxReducer,
    Reducer,
    ReducerCall,
    SumReducer,
    online_softmax,
)
from .reducer import sum  # noqa: A004

__version__ = "0.1.0"

__all__ = [
    "CompiledVariant",
    "Graph",
    "GraphSchema",
    "Kernel",
    "MessagePassing",
    "OnlineSoftmaxItem",
    "OnlineSoftmaxReducer",
    "Reducer",
    "ReducerCall",
    "SumReducer",
    "__version__",
    "config",
    "interop",
    "nn",
    "online_softmax",
    "reducer",
    "sum",
]
