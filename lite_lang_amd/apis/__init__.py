"""Streaming HTTP front end of the token loop (counterpart of litelang/apis/).

`HttpServerManager` runs the continuous-batching `Scheduler` in a thread of
its own and turns each request's output queue into a generator;
`api_server.app` is the FastAPI application with the reference's two routes
(`POST /generate`, `POST /generate_stream`) and request body.
"""
from .http_server_manager import HttpServerManager, RequestRefused

__all__ = ["HttpServerManager", "RequestRefused"]
