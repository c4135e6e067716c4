"""`/v1/systemone` HTTP serving on the HIP decision path (`python -m deciax_amd.serve --impl hip`)."""

from deciax_amd.serve.wsgi import DecisionApp, Reply, make_server, serve

__all__ = ["DecisionApp", "Reply", "make_server", "serve"]
