"""`/v1/systemone` HTTP serving on the HIP decision path (`python -m deciax_amd.serve --impl hip`)."""

from deciax_amd.serve.app import Response, Service, make_server, serve

__all__ = ["Response", "Service", "make_server", "serve"]
