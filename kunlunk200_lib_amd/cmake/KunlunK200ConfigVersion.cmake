# Version 0.7.12 (the reference release whose interface this library keeps),
# compatible with any request of the same major version that is not newer.
set(PACKAGE_VERSION "0.7.12")
if(PACKAGE_FIND_VERSION_MAJOR STREQUAL "0" AND NOT PACKAGE_FIND_VERSION VERSION_GREATER PACKAGE_VERSION)
    set(PACKAGE_VERSION_COMPATIBLE TRUE)
    if(PACKAGE_FIND_VERSION VERSION_EQUAL PACKAGE_VERSION)
        set(PACKAGE_VERSION_EXACT TRUE)
    endif()
else()
    set(PACKAGE_VERSION_COMPATIBLE FALSE)
endif()
# a 64-bit library: a project without a language (no pointer size) is not checked
if(DEFINED CMAKE_SIZEOF_VOID_P AND NOT CMAKE_SIZEOF_VOID_P STREQUAL "" AND NOT CMAKE_SIZEOF_VOID_P STREQUAL "8")
    set(PACKAGE_VERSION "${PACKAGE_VERSION} (64-bit only)")
    set(PACKAGE_VERSION_UNSUITABLE TRUE)
endif()
